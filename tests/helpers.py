"""Shared test helpers: tensor conversion and the parity bars."""
import numpy as np
import torch

# bf16 output tolerance for the attention paths (max abs, mean abs), fp32 accumulation.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3
# The absolute bar alone cannot fail at the full decode sizes: a softmax over
# 8192 flat N(0,1) scores averages the values down to |out| ~ 5e-3, so losing a
# whole V tile moves the output by less than MEAN_ABS.  Every comparison also
# bounds the error relative to the output, ||actual - expected||_2 /
# ||expected||_2 <= REL_L2: bf16 rounding of the output alone gives about
# 2^-9 / sqrt(3) ~ 1.1e-3 (tests/test_parity_bar.py checks that planted
# mistakes of that kind fail it and the rounded exact result passes).
REL_L2 = 1e-2


def to_np(t):
    return t.detach().to(torch.float32).cpu().numpy().astype(np.float64)


def bits(t):
    """bf16 tensor -> uint16 numpy bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def rel_l2(actual, expected):
    """||actual - expected||_2 / ||expected||_2 (0 when both are all zeros,
    inf when only the expected result is)."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    num, den = np.linalg.norm((actual - expected).ravel()), np.linalg.norm(expected.ravel())
    if den == 0.0:
        return 0.0 if num == 0.0 else np.inf
    return num / den


def assert_close(actual, expected, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what='', rel=REL_L2):
    """The absolute bar (max, mean) and the output-relative bar rel_l2 <= rel."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    assert np.isfinite(actual).all(), f'{what}: non-finite output'
    err = np.abs(actual - expected)
    r = rel_l2(actual, expected)
    if what:
        print(f'{what}: max abs err {err.max():.3e}, mean abs err {err.mean():.3e}, rel l2 {r:.3e}', flush=True)
    assert err.max() <= max_abs, f'{what}: max abs err {err.max():.3e} > {max_abs}'
    assert err.mean() <= mean_abs, f'{what}: mean abs err {err.mean():.3e} > {mean_abs}'
    if rel is not None:
        assert r <= rel, f'{what}: relative l2 err {r:.3e} > {rel}'
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
