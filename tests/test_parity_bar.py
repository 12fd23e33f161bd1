"""The parity bar itself, on the CPU: at the full latent decode size (one
sequence of the batch-16 32K layer -- 8192 beacon rows of rank 32 per KV head,
4 sinks + 128 tail + the current token, 32/8 heads, N(0,1) inputs as the
benchmark draws them) the output-relative bound of tests.helpers passes the
reference's own bf16 result and fails planted kernel-sized mistakes that the
absolute bound (max 2e-2, mean 2e-3) lets through.

The planted mistakes are made in the oracle's inputs, as a lost tile or a
wrong head index in a kernel would show in its output:
  * the V rows of the last eighth of the beacons read as zeros (a lost split),
  * one KV head's V up-projection block taken from its neighbour (a wrong
    head index in the lift).
Each is tried with the benchmark's flat queries and with queries twice as
large (a peaked softmax: the golden fixtures' queries are about 2.3 times
their keys)."""
import numpy as np
import pytest

from oracle import attention as oa
from tests.helpers import MAX_ABS, MEAN_ABS, REL_L2, assert_close, rel_l2

HQ, HKV, D, RANK, BEACONS, RAW = 32, 8, 128, 32, 8192, 133


def _orthonormal(rng, rows, cols):
    q, r = np.linalg.qr(rng.standard_normal((rows, cols)))
    return q * np.sign(np.diag(r))[None]


def _bases(rng):
    w = np.zeros((HKV * D, HKV * RANK))
    for h in range(HKV):
        w[h * D:(h + 1) * D, h * RANK:(h + 1) * RANK] = _orthonormal(rng, D, RANK)
    return w


@pytest.fixture(scope='module')
def layer():
    """One C1-sized sequence (B = 2), bf16-exact N(0,1) draws."""
    from oracle.bf16 import round_bf16
    rng = np.random.Generator(np.random.PCG64(31))
    B = 2
    r = lambda *s: round_bf16(rng.standard_normal(s)).astype(np.float64)
    return dict(q=r(B, HQ, 1, D), raw_k=r(B, HKV, RAW, D), raw_v=r(B, HKV, RAW, D),
                lat_k=r(B, 1, BEACONS, HKV * RANK), lat_v=r(B, 1, BEACONS, HKV * RANK),
                up_k=round_bf16(_bases(rng)).astype(np.float64), up_v=round_bf16(_bases(rng)).astype(np.float64))


def _run(L, q_scale=1.0, bf16=True, **over):
    a = dict(L, **over)
    out, _ = oa.latent_layer(a['q'] * q_scale, a['raw_k'], a['raw_v'], a['lat_k'], a['lat_v'], a['up_k'],
                             a['up_v'], D ** -0.5, HKV, bf16_boundaries=bf16)
    return out


def _lost_tile(L):
    v = L['lat_v'].copy()
    v[:, :, BEACONS - BEACONS // 8:] = 0.0
    return dict(lat_v=v)


def _swapped_head(L):
    w = L['up_v'].copy()
    h, n = 3, 4
    w[h * D:(h + 1) * D, h * RANK:(h + 1) * RANK] = L['up_v'][n * D:(n + 1) * D, n * RANK:(n + 1) * RANK]
    return dict(up_v=w)


@pytest.mark.parametrize('q_scale', [1.0, 2.0])
def test_reference_rounding_passes_the_bar(layer, q_scale):
    """The reference's bf16 path (its roundings of the branch outputs, the
    absorbed query and the lift) against the float64 result: well inside
    every bound, so the bound leaves room for a correct kernel."""
    exact = _run(layer, q_scale, bf16=False)
    ref = _run(layer, q_scale, bf16=True)
    assert rel_l2(ref, exact) < REL_L2 / 2
    assert_close(ref, exact, what=f'reference bf16 rounding, q x{q_scale}')


@pytest.mark.parametrize('q_scale', [1.0, 2.0])
@pytest.mark.parametrize('mistake', [_lost_tile, _swapped_head])
def test_planted_mistakes_fail_the_relative_bound(layer, mistake, q_scale):
    ref = _run(layer, q_scale)
    bad = _run(layer, q_scale, **mistake(layer))
    r = rel_l2(bad, ref)
    err = np.abs(bad - ref)
    print(f'{mistake.__name__} q x{q_scale}: max {err.max():.3e} mean {err.mean():.3e} rel {r:.3e}')
    assert r > 5 * REL_L2, f"{mistake.__name__}: relative error {r:.3e} is not well above the bound"
    with pytest.raises(AssertionError, match='relative l2'):
        assert_close(bad, ref, max_abs=np.inf, mean_abs=np.inf)


def test_lost_tile_passes_the_absolute_bar_alone(layer):
    """Why the relative bound exists: at flat N(0,1) inputs a lost eighth of
    the V rows stays inside the absolute bar."""
    ref = _run(layer)
    bad = _run(layer, **_lost_tile(layer))
    err = np.abs(bad - ref)
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS
