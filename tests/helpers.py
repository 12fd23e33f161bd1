"""Shared test helpers: tensor conversion and the parity bars."""
import numpy as np
import torch

# bf16 output tolerance for the attention paths (max abs, mean abs), fp32 accumulation.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def to_np(t):
    return t.detach().to(torch.float32).cpu().numpy().astype(np.float64)


def bits(t):
    """bf16 tensor -> uint16 numpy bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def assert_close(actual, expected, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what=''):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    assert np.isfinite(actual).all(), f'{what}: non-finite output'
    err = np.abs(actual - expected)
    assert err.max() <= max_abs, f'{what}: max abs err {err.max():.3e} > {max_abs}'
    assert err.mean() <= mean_abs, f'{what}: mean abs err {err.mean():.3e} > {mean_abs}'
    return err.max(), err.mean()


def assert_lse_close(actual, expected, atol=2e-3, what=''):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    inf_a, inf_e = np.isneginf(actual), np.isneginf(expected)
    assert (inf_a == inf_e).all(), f'{what}: -inf LSE rows differ'
    fin = ~inf_e
    if fin.any():
        err = np.abs(actual[fin] - expected[fin]).max()
        assert err <= atol, f'{what}: LSE err {err:.3e} > {atol}'
