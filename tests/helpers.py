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
    if what:
        print(f'{what}: max abs err {err.max():.3e}, mean abs err {err.mean():.3e}', flush=True)
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


def neighbour_of_exact(actual, exact, rounded, abs_terms):
    """Every bf16 output is one of the two bf16 neighbours of the float64 GEMM
    result up to the fp32 accumulation error (any fp32-accumulating GEMM -- this
    kernel or hipBLASLt -- can land on either side of a near-tie, and near a
    cancellation the error is absolute), and almost all equal its correct
    rounding.  abs_terms: the GEMM of absolute values (sum |w||x|)."""
    a, x = np.asarray(actual, np.float64), np.asarray(exact, np.float64)
    mag = np.maximum(np.abs(x), 1e-30)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 7)
    accumulation = np.asarray(abs_terms, np.float64) * 2.0 ** -20
    err = np.abs(a - x)
    bad = err >= ulp * 1.0001 + accumulation
    assert not bad.any(), list(zip(a[bad][:4], x[bad][:4]))
    assert (a == np.asarray(rounded, np.float64)).mean() > 0.98
