"""Golden fixtures of the attention hot path: seeded inputs, the oracle's results.

Inputs are drawn with numpy's PCG64 as small integers times a power of two, so
every value is exact in bf16 and no transcendental function takes part: any
host draws the same bits.  RoPE tables come from float64 angles through
Python's cos/sin, rounded to fp32 (the tables' own rounding rule is pinned by
the RoPE tests; here both sides only have to read the same table).  A fixture
file `<case>.npz` holds

  * `sha_<input>`: SHA-256 of each input's bits as drawn here (bf16 bits for
    bf16 tensors, fp32 bytes for tables, int64 for indices) -- a host that
    draws other bits fails loudly instead of comparing other inputs;
  * `sha_<result>`: SHA-256 of the bits of every bit-exact result (RoPE'd
    queries and keys, page gathers);
  * every floating-point result as float32 (bf16-rounded results exactly;
    the exact down-projection GEMM in float64), and integer index vectors
    as int64.

    python tests/golden/make_golden.py      # rewrite tests/golden/*.npz

Cases (the reference call each one restates is cited in its builder):
  c0_latent_decode   B1, 32/8 heads, head_dim 128, 4 sinks + 124 tail + current
                     token, 992 beacons of rank 32 per KV head (R 256) --
                     the reference's CPU-runnable decode shape
  c2_recon_decode    reconstruction decode, 40/8 heads, B2, 256 beacons with
                     K-RoPE at their slot positions
  c3_prefill_window  one prefill window: 4 sinks, 16 history beacons, 128 raw
                     + 32 beacon rows, 2/1 heads; beacon latents of the window
  c4_paged_decode    paged decode over BeaconPageLayout(16, 8, 64, 64, 256)
                     pages and 16-token raw pages, 4 sequences (0-100 beacons)
"""
import hashlib
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import attention as oa          # noqa: E402
from oracle import paged as opaged          # noqa: E402
from oracle import rope as orope            # noqa: E402
from oracle.bf16 import round_bf16, to_bits  # noqa: E402

CASES = ('c0_latent_decode', 'c2_recon_decode', 'c3_prefill_window', 'c4_paged_decode')
SEEDS = dict(c0_latent_decode=1000, c2_recon_decode=1002, c3_prefill_window=1003, c4_paged_decode=1004)
D = 128
THETA = 500000.0


def path(case):
    return os.path.join(HERE, case + '.npz')


def _ints(rng, shape, span=64, shift=5):
    """Integers uniform in [-span, span] times 2**-shift (exact in bf16 for
    span <= 256).  Queries take shift 4 (values in [-4, 4]) so that the
    softmax is peaked rather than flat."""
    return (rng.integers(-span, span + 1, size=shape) * 2.0 ** -shift).astype(np.float32)


def _bases(rng, kv_heads, rank):
    """Block-diagonal up-projection [kv_heads*D, kv_heads*rank] in nn.Linear
    layout, per-KV-head blocks of k/64 with k in [-16, 16]."""
    w = np.zeros((kv_heads * D, kv_heads * rank), np.float32)
    for h in range(kv_heads):
        w[h * D:(h + 1) * D, h * rank:(h + 1) * rank] = _ints(rng, (D, rank), 16, 6)
    return w


def rope_table(rows, dim=D, base=THETA):
    """(cos, sin) [rows, dim] fp32; each row is its first half twice, as the
    rotary embedding's tables are (modeling_utils.py:359-376)."""
    inv = [base ** (-(2.0 * i) / dim) for i in range(dim // 2)]
    cos = np.empty((rows, dim // 2), np.float64)
    sin = np.empty((rows, dim // 2), np.float64)
    for p in range(rows):
        for i, f in enumerate(inv):
            cos[p, i] = math.cos(p * f)
            sin[p, i] = math.sin(p * f)
    cos, sin = cos.astype(np.float32), sin.astype(np.float32)
    return np.concatenate([cos, cos], 1), np.concatenate([sin, sin], 1)


def sha_bf16(x):
    """SHA-256 of the bf16 bits of x (values that are bf16 already)."""
    bits = to_bits(x)
    return hashlib.sha256(np.ascontiguousarray(bits).tobytes()).hexdigest()


def input_digests(inputs):
    """sha_<name> of every input: bf16 bits for the bf16 tensors (float32
    arrays here), raw bytes for tables (fp32) and integer arrays."""
    out = {}
    for name, x in inputs.items():
        if name in ('cos', 'sin'):
            out[name] = hashlib.sha256(np.ascontiguousarray(x, np.float32).tobytes()).hexdigest()
        elif isinstance(x, np.ndarray) and x.dtype == np.float32:
            out[name] = sha_bf16(x)
        elif isinstance(x, np.ndarray):
            out[name] = hashlib.sha256(np.ascontiguousarray(x, np.int64).tobytes()).hexdigest()
    return out


# ----------------------------------------------------------------------------- C0

def c0_inputs():
    """fa2_decode.decode's call at the reference's CPU-runnable shape
    (fa2_decode.py:77-166): q [1,1,32,128] unrotated at position 4096, raw
    K/V [1,129,8,128] (4 sinks at 0..3, tail 3972..4095, current token 4096;
    K unrotated, rotated by fused_rope, decode_ops.py:14-31), beacon latents
    [1,992,256] with no RoPE, block-diagonal bases [1024,256]."""
    rng = np.random.Generator(np.random.PCG64(SEEDS['c0_latent_decode']))
    B, H, HKV, r, S, T, NB, CTX = 1, 32, 8, 32, 4, 124, 992, 4096
    inp = dict(q=_ints(rng, (B, 1, H, D), 64, 4), raw_k=_ints(rng, (B, S + T + 1, HKV, D)),
               raw_v=_ints(rng, (B, S + T + 1, HKV, D)), lat_k=_ints(rng, (B, NB, HKV * r)),
               lat_v=_ints(rng, (B, NB, HKV * r)), up_k=_bases(rng, HKV, r), up_v=_bases(rng, HKV, r))
    inp['cos'], inp['sin'] = rope_table(CTX + 1)
    inp['q_positions'] = np.full((B, 1), CTX, np.int64)
    inp['raw_indices'] = np.arange(T, dtype=np.int64)          # tail slot s -> raw_indices[s-S] + S + history
    meta = dict(kv_heads=HKV, sink=S, history=CTX - T - S, scale=D ** -0.5)
    return inp, meta


def c0_expected(inp, meta):
    q = inp['q'].transpose(0, 2, 1, 3)                          # [B, H, 1, D]
    k = inp['raw_k'].transpose(0, 2, 1, 3)                      # [B, Hkv, N, D]
    q_rot, k_rot = orope.rope_decode(q, k, inp['cos'], inp['sin'], inp['q_positions'], inp['raw_indices'],
                                     meta['sink'], meta['history'])
    out, lse = oa.latent_layer(q_rot.astype(np.float64), k_rot.astype(np.float64),
                               inp['raw_v'].transpose(0, 2, 1, 3).astype(np.float64),
                               inp['lat_k'][:, None].astype(np.float64), inp['lat_v'][:, None].astype(np.float64),
                               inp['up_k'].astype(np.float64), inp['up_v'].astype(np.float64), meta['scale'],
                               meta['kv_heads'])
    return dict(sha_q_rot=sha_bf16(q_rot), sha_k_rot=sha_bf16(k_rot), out=out, lse=lse)


# ----------------------------------------------------------------------------- C2

def c2_inputs():
    """LlamaAttention.forward with the reconstruction backend
    (modeling_llama.py:1402-1483) at the Qwen2.5-14B attention shape: q
    [2,1,40,128] unrotated at position 388, raw K (rotated cache rows) / V
    [2,133,8,128], beacon latents [2,256,256] whose rebuilt keys are rotated
    at slot positions 4..259, block-diagonal bases."""
    rng = np.random.Generator(np.random.PCG64(SEEDS['c2_recon_decode']))
    B, H, HKV, r, S, T, NB = 2, 40, 8, 32, 4, 128, 256
    ctx = S + NB + T
    inp = dict(q=_ints(rng, (B, 1, H, D), 64, 4), raw_k=_ints(rng, (B, S + T + 1, HKV, D)),
               raw_v=_ints(rng, (B, S + T + 1, HKV, D)), lat_k=_ints(rng, (B, NB, HKV * r)),
               lat_v=_ints(rng, (B, NB, HKV * r)), up_k=_bases(rng, HKV, r), up_v=_bases(rng, HKV, r))
    inp['cos'], inp['sin'] = rope_table(ctx + 1)
    inp['q_positions'] = np.full((B, 1), ctx, np.int64)
    inp['beacon_positions'] = np.broadcast_to(S + np.arange(NB, dtype=np.int64), (B, NB)).copy()
    return inp, dict(kv_heads=HKV, scale=D ** -0.5)


def c2_expected(inp, meta):
    """Float64 attention over [rebuilt, rotated beacons ; raw rows]: keys as the
    reference builds them (bf16 up-projection, then its bf16 RoPE steps:
    llama3/memory.py:29-36, modeling_llama.py:1108-1216) and as the fused
    route's fp32 rotation (exact rebuild, rotated, one bf16 rounding)."""
    HKV, scale = meta['kv_heads'], meta['scale']
    cos, sin = inp['cos'], inp['sin']
    q = inp['q'].transpose(0, 2, 1, 3)
    q_rot = orope.rotate_bf16(q, cos[inp['q_positions'][0, 0]][None], sin[inp['q_positions'][0, 0]][None])
    lat_k = inp['lat_k'][:, None].astype(np.float64)
    lat_v = inp['lat_v'][:, None].astype(np.float64)
    rv = oa.reconstruct(lat_v, inp['up_v'].astype(np.float64), None, HKV, D)
    raw_k = inp['raw_k'].transpose(0, 2, 1, 3).astype(np.float64)
    raw_v = inp['raw_v'].transpose(0, 2, 1, 3).astype(np.float64)
    bp = inp['beacon_positions'][0]
    c_rows, s_rows = cos[bp][None], sin[bp][None]
    rk = oa.reconstruct(lat_k, inp['up_k'].astype(np.float64), None, HKV, D)
    ref_keys = orope.rotate_bf16(rk.astype(np.float32), c_rows, s_rows).astype(np.float64)
    xk = oa.reconstruct(lat_k, inp['up_k'].astype(np.float64), None, HKV, D, bf16_boundaries=False)
    c64, s64 = round_bf16(c_rows).astype(np.float64), round_bf16(s_rows).astype(np.float64)
    fp32_keys = round_bf16(xk * c64 + orope.rotate_half(xk) * s64).astype(np.float64)
    res = {}
    for name, keys in (('reference', ref_keys), ('fp32', fp32_keys)):
        k = np.concatenate([keys, raw_k], axis=2)
        v = np.concatenate([rv, raw_v], axis=2)
        out, lse = oa.eager_forward(q_rot.astype(np.float64).transpose(0, 2, 1, 3), k.transpose(0, 2, 1, 3),
                                    v.transpose(0, 2, 1, 3), scale)
        res[f'out_{name}'], res[f'lse_{name}'] = out, lse        # out [B, 1, H, D], lse [B, H, 1]
    return res


# ----------------------------------------------------------------------------- C3

def c3_inputs():
    """One join-prefill window (modeling_llama.py:1632-1809): keys [sink (4) ;
    rebuilt history (16 beacons) ; window (160 rows, every fifth a beacon
    row)], positions 0..179, q for the window's rows; fused_prefill_rope leaves
    history and window beacon keys unrotated (prefill_ops.py:48-73); the
    window's beacon rows are down-projected to K latents (modeling_llama.py:
    383-390) from hidden [1,160,256] with a [32, 256] weight."""
    rng = np.random.Generator(np.random.PCG64(SEEDS['c3_prefill_window']))
    B, H, HKV, S, NH, L, HID, R = 1, 2, 1, 4, 16, 160, 256, 32
    N = S + NH + L
    roles = np.zeros(L, np.int64)
    roles[4::5] = 1
    inp = dict(q=_ints(rng, (B, L, H, D), 64, 4), k=_ints(rng, (B, N, HKV, D)), v=_ints(rng, (B, N, HKV, D)),
               hidden=_ints(rng, (B, L, HID), 64, 6), down=_ints(rng, (R, HID), 16, 8))
    inp['cos'], inp['sin'] = rope_table(N)
    inp['positions'] = np.broadcast_to(np.arange(N, dtype=np.int64), (B, N)).copy()
    inp['roles'] = roles
    inp['beacon_rows'] = np.nonzero(roles)[0].astype(np.int64)
    return inp, dict(sink=S, scale=D ** -0.5)


def c3_expected(inp, meta):
    q = inp['q'].transpose(0, 2, 1, 3)
    k = inp['k'].transpose(0, 2, 1, 3)
    q_rot, k_rot = orope.prefill_rope(q, k, inp['cos'], inp['sin'], inp['positions'], inp['roles'], meta['sink'])
    out, lse = oa.eager_forward(q_rot.astype(np.float64).transpose(0, 2, 1, 3),
                                k_rot.astype(np.float64).transpose(0, 2, 1, 3), inp['v'].astype(np.float64),
                                meta['scale'], causal=True)
    latents = oa.down_project(inp['hidden'].astype(np.float64), inp['down'].astype(np.float64),
                              inp['beacon_rows'], bf16_boundaries=False)
    return dict(sha_q_rot=sha_bf16(q_rot), sha_k_rot=sha_bf16(k_rot), out=out, lse=lse, latents=latents)


# ----------------------------------------------------------------------------- C4

C4_LAYOUT = (16, 8, 64, 64, 256)          # raw_block_size, token_ratio, key_rank, value_rank, raw_width


def c4_inputs():
    """The vLLM plugin's paged decode (paged_model.py:36-52 -> paged_cache.py:
    60-87 -> fa2_decode.py:77-166): 4 sequences with 0 / 7 / 33 / 100 beacons
    in BeaconPageLayout(16, 8, 64, 64, 256) pages of a 96-page pool at a seeded
    permutation, sinks + tail + current token (5 / 10 / 22 / 45 rows) in
    16-token raw pages; q [4,1,8,128] already rotated, 8/2 heads, rank 32 per
    KV head."""
    rng = np.random.Generator(np.random.PCG64(SEEDS['c4_paged_decode']))
    layout = opaged.Layout(*C4_LAYOUT)
    HQ, HKV, r, POOL = 8, 2, 32, 96
    nb = np.array([0, 7, 33, 100], np.int64)
    raw = np.array([5, 10, 22, 45], np.int64)
    need = (nb + layout.slots - 1) // layout.slots
    perm = rng.permutation(POOL)
    tables = np.zeros((len(nb), int(need.max())), np.int64)
    off = 0
    for s, n in enumerate(need):
        tables[s, :n] = perm[off:off + n]
        off += n
    raw_blocks = int((raw.max() + 15) // 16)
    raw_tables = rng.permutation(len(nb) * raw_blocks).reshape(len(nb), raw_blocks).astype(np.int64)
    inp = dict(pool=_ints(rng, (POOL, layout.page_elements)),
               raw_pool=_ints(rng, (len(nb) * raw_blocks, 16, 2, HKV, D)),
               q=_ints(rng, (len(nb), 1, HQ, D), 64, 4), up_k=_bases(rng, HKV, r), up_v=_bases(rng, HKV, r),
               tables=tables, raw_tables=raw_tables, lat_len=nb, raw_len=raw)
    return inp, dict(kv_heads=HKV, scale=D ** -0.5)


def c4_gather(inp):
    """Beacon rows [B, max nb, width] and raw rows [B, max raw, 2, Hkv, D] at
    the oracle's page indices, zero past each sequence, plus the index vectors."""
    layout = opaged.Layout(*C4_LAYOUT)
    nb, raw = inp['lat_len'], inp['raw_len']
    rows = np.zeros((len(nb), int(nb.max()), layout.width), np.float32)
    raws = np.zeros((len(nb), int(raw.max())) + inp['raw_pool'].shape[2:], np.float32)
    idx = {}
    for b, (n, m) in enumerate(zip(nb, raw)):
        page, first = opaged.beacon_indices(layout, inp['tables'][b], 0, int(n))
        rows[b, :n] = inp['pool'][page[:, None], first[:, None] + np.arange(layout.width)[None]]
        blk, offs = opaged.raw_indices(16, inp['raw_tables'][b], 0, int(m))
        raws[b, :m] = inp['raw_pool'][blk, offs]
        idx[f'beacon_page_{b}'], idx[f'beacon_column_{b}'] = page, first
        idx[f'raw_block_{b}'], idx[f'raw_offset_{b}'] = blk, offs
    return rows, raws, idx


def c4_expected(inp, meta):
    layout = opaged.Layout(*C4_LAYOUT)
    rows, raws, idx = c4_gather(inp)
    res = dict(idx)
    res['sha_beacon_rows'] = sha_bf16(rows)
    res['sha_raw_rows'] = sha_bf16(raws)
    outs, lses = [], []
    for b, (n, m) in enumerate(zip(inp['lat_len'], inp['raw_len'])):
        lat = rows[b:b + 1, :n].astype(np.float64)
        out, lse = oa.latent_layer(inp['q'][b:b + 1].transpose(0, 2, 1, 3).astype(np.float64),
                                   raws[b:b + 1, :m, 0].transpose(0, 2, 1, 3).astype(np.float64),
                                   raws[b:b + 1, :m, 1].transpose(0, 2, 1, 3).astype(np.float64),
                                   lat[:, None, :, :layout.key_rank], lat[:, None, :, layout.key_rank:],
                                   inp['up_k'].astype(np.float64), inp['up_v'].astype(np.float64), meta['scale'],
                                   meta['kv_heads'])
        outs.append(out)
        lses.append(lse)
    res['out'] = np.concatenate(outs)                              # [B, H, 1, D]
    res['lse'] = np.concatenate(lses)                              # [B, H, 1]
    return res


# results kept in float64: the down-projection's exact GEMM, against which a
# bf16 result is checked to one rounding
FLOAT64 = ('latents',)

BUILDERS = dict(c0_latent_decode=(c0_inputs, c0_expected), c2_recon_decode=(c2_inputs, c2_expected),
                c3_prefill_window=(c3_inputs, c3_expected), c4_paged_decode=(c4_inputs, c4_expected))


def build(case):
    """(inputs, meta, expected) of one case, expected including sha_<input> digests."""
    make_inputs, make_expected = BUILDERS[case]
    inp, meta = make_inputs()
    exp = make_expected(inp, meta)
    exp.update({f'sha_{k}': v for k, v in input_digests(inp).items()})
    return inp, meta, exp


def load(case):
    with np.load(path(case), allow_pickle=False) as f:
        return {k: (str(f[k]) if f[k].dtype.kind == 'U' else f[k]) for k in f.files}


def write(case):
    _, _, exp = build(case)
    arrays = {}
    for k, v in exp.items():
        if isinstance(v, str):
            arrays[k] = np.array(v)
        elif np.asarray(v).dtype.kind == 'f':
            arrays[k] = np.asarray(v, np.float64 if k in FLOAT64 else np.float32)
        else:
            arrays[k] = np.asarray(v, np.int64)
    np.savez_compressed(path(case), **arrays)


if __name__ == '__main__':
    for c in sys.argv[1:] or CASES:
        write(c)
        print(c, os.path.getsize(path(c)), 'bytes')
