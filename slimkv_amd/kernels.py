"""Tensor-level calls into the HIP library (device memory and streams via torch).

Each function validates its tensors, allocates outputs and the workspace from
torch's caching allocator (so the calls are HIP-graph capturable), fills the C
argument struct and enqueues on torch's current stream.  Nothing here computes
on the CPU.
"""
import ctypes
import math

import torch

from . import _lib
from ._lib import check, lib

BF16 = torch.bfloat16


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _need_device(*tensors):
    for t in tensors:
        if t is not None and t.device.type != 'cuda':
            raise ValueError('slimkv_amd kernels need device tensors (no CPU path)')


def _need_bf16(*tensors):
    for t in tensors:
        if t is not None and t.dtype != BF16:
            raise ValueError(f'expected bfloat16, found {t.dtype}')


def _last_contiguous(t):
    return t if t.stride(-1) == 1 else t.contiguous()


def _workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def attention_forward(q, k, v, scale, causal=False, splits=0, seqlens=None, out=None, lse=None):
    """BSHD split-K attention.  q [B,Lq,Hq,Wk], k [B,N,Hk,Wk], v [B,N,Hk,Wv].

    Returns (out [B,Lq,Hq,Wv] bf16, lse [B,Hq,Lq] fp32).
    """
    _need_device(q, k, v, seqlens)
    _need_bf16(q, k, v)
    q, k, v = (_last_contiguous(x) for x in (q, k, v))
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError('BSHD tensors required')
    B, Lq, Hq, Wk = q.shape
    _, N, Hk, _ = k.shape
    Wv = v.shape[-1]
    if k.shape[0] != B or k.shape[-1] != Wk or v.shape[:3] != k.shape[:3]:
        raise ValueError('invalid K/V shapes')
    if out is None:
        out = torch.empty(B, Lq, Hq, Wv, dtype=BF16, device=q.device)
    if lse is None:
        lse = torch.empty(B, Hq, Lq, dtype=torch.float32, device=q.device)
    if seqlens is not None:
        if seqlens.dtype != torch.int32 or not seqlens.is_contiguous() or seqlens.numel() != B:
            raise ValueError('One int32 cache length per sequence required')
    a = _lib.AttentionArgs(
        _ptr(q), *q.stride()[:3], _ptr(k), *k.stride()[:3], _ptr(v), *v.stride()[:3],
        _ptr(out), *out.stride()[:3], _ptr(lse), _ptr(seqlens),
        B, Lq, Hq, Hk, N, Wk, Wv, float(scale), int(bool(causal)), int(splits))
    nbytes = lib().slimkv_attention_workspace(ctypes.byref(a))
    if nbytes == 0:
        check(-1)
    ws = _workspace(nbytes, q.device)
    check(lib().slimkv_attention_forward(ctypes.byref(a), _ptr(ws), nbytes, _lib.stream_handle(q.device)))
    return out, lse


def prefill_attention(q, k, v, scale, causal=True, seqlens_k=None, out=None, lse=None, *, q_positions=None,
                      cos=None, sin=None):
    """Causal (bottom-right) GQA prefill attention, head_dim 128 (MFMA flash
    attention).  q [B,Lq,Hq,128], k/v [B,N,Hk,128] BSHD bf16.  With fp32
    RoPE tables cos/sin [rows, 128] and q_positions [B, >= Lq] the kernel
    rotates each query row as it loads it (the bits of prefill_rope's query
    rotation), reading (bf16 cos | bf16 sin) pairs prepared once per table
    (prepare_rope_pairs, cached on the table); k is taken as given.

    Returns (out [B,Lq,Hq,128] bf16, lse [B,Hq,Lq] fp32).
    """
    _need_device(q, k, v, seqlens_k, q_positions, cos, sin)
    _need_bf16(q, k, v)
    q, k, v = (_last_contiguous(x) for x in (q, k, v))
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError('BSHD tensors required')
    B, Lq, Hq, D = q.shape
    _, N, Hk, _ = k.shape
    if k.shape[0] != B or k.shape[-1] != D or v.shape != k.shape:
        raise ValueError('invalid K/V shapes')
    if out is None:
        out = torch.empty(B, Lq, Hq, D, dtype=BF16, device=q.device)
    if lse is None:
        lse = torch.empty(B, Hq, Lq, dtype=torch.float32, device=q.device)
    if seqlens_k is not None:
        if seqlens_k.dtype != torch.int32 or not seqlens_k.is_contiguous() or seqlens_k.numel() != B:
            raise ValueError('One int32 key length per sequence required')
    rope, pairs = (None, 0, 0, None, 0), None
    if cos is not None:
        if sin is None or q_positions is None:
            raise ValueError('query RoPE needs cos, sin and q_positions')
        if cos.dim() != 2 or cos.shape[1] != D:
            raise ValueError('RoPE tables must be fp32 [rows, head_dim]')
        pairs, repeats = prepare_rope_pairs(cos, sin)
        q_positions = q_positions.to(torch.int64)
        if q_positions.stride(-1) != 1:
            q_positions = q_positions.contiguous()
        if q_positions.dim() != 2 or q_positions.shape[0] != B or q_positions.shape[1] < Lq:
            raise ValueError('q_positions must be [B, >= Lq]')
        rope = (_ptr(pairs), pairs.shape[0], int(repeats), _ptr(q_positions), q_positions.stride(0))
    a = _lib.PrefillAttentionArgs(
        _ptr(q), *q.stride()[:3], _ptr(k), *k.stride()[:3], _ptr(v), *v.stride()[:3],
        _ptr(out), *out.stride()[:3], _ptr(lse), _ptr(seqlens_k),
        B, Lq, Hq, Hk, N, D, float(scale), int(bool(causal)), *rope)
    check(lib().slimkv_prefill_attention(ctypes.byref(a), _lib.stream_handle(q.device)))
    return out, lse


def down_project(x, weight, rows=None, *, blocks=1, out=None):
    """Latents of selected rows: out[b, i] = bf16(x[b, rows[i]] @ weight^T).

    x [B, L, K] bf16, weight [N, K] (nn.Linear layout), rows int64 [n] or None
    (all rows).  `blocks` > 1 declares a block-diagonal weight.  Returns
    out [B, n, N] bf16.
    """
    a, out, keep = _down_args(x, weight, rows, blocks, out)
    nbytes = lib().slimkv_down_project_workspace(ctypes.byref(a))
    if nbytes == 0:
        check(-1)
    ws = _workspace(nbytes, out.device)
    check(lib().slimkv_down_project(ctypes.byref(a), _ptr(ws), nbytes, _lib.stream_handle(out.device)))
    return out


def down_project_pair(first, second):
    """Two down-projections in one launch where the library can (the K and V
    latents of a window's beacon rows), the same bits as two down_project
    calls.  `first` / `second`: dicts of down_project's arguments (x, weight,
    rows, blocks, out).  Returns the two outputs."""
    names = ('x', 'weight', 'rows', 'blocks', 'out')
    for kw in (first, second):
        if set(kw) - set(names):
            raise TypeError(f'unknown down_project arguments {sorted(set(kw) - set(names))}')
    a, out_a, keep_a = _down_args(first['x'], first['weight'], first.get('rows'), first.get('blocks', 1),
                                  first.get('out'))
    b, out_b, keep_b = _down_args(second['x'], second['weight'], second.get('rows'), second.get('blocks', 1),
                                  second.get('out'))
    if out_a.device != out_b.device:
        raise ValueError('both down-projections must be on one device')
    nbytes = lib().slimkv_down_project_pair_workspace(ctypes.byref(a), ctypes.byref(b))
    if nbytes == 0:
        check(-1)
    ws = _workspace(nbytes, out_a.device)
    check(lib().slimkv_down_project_pair(ctypes.byref(a), ctypes.byref(b), _ptr(ws), nbytes,
                                         _lib.stream_handle(out_a.device)))
    return out_a, out_b


def _down_args(x, weight, rows, blocks, out):
    """The slimkv_down_project_args of one down-projection, its output and the
    tensors the arguments point into."""
    _need_device(x, weight, rows)
    _need_bf16(x, weight)
    if x.dim() != 3 or weight.dim() != 2 or weight.shape[1] != x.shape[2]:
        raise ValueError('x must be [B, L, K] and weight [N, K]')
    x = _last_contiguous(x)
    weight = weight.contiguous()
    B, L, K = x.shape
    N = weight.shape[0]
    if rows is not None:
        rows = rows.to(dtype=torch.long).contiguous()
    n = L if rows is None else rows.numel()
    if out is None:
        out = torch.empty(B, n, N, dtype=BF16, device=x.device)
    if out.shape != (B, n, N) or out.stride(2) != 1:
        raise ValueError('out must be [B, n, N] with contiguous rows')
    a = _lib.DownProjectArgs(_ptr(x), x.stride(0), x.stride(1), _ptr(rows), n, L, _ptr(weight),
                             _ptr(out), out.stride(0), out.stride(1), B, K, N, int(blocks))
    return a, out, (x, weight, rows, out)


def down_project_to_pages(x, weight, pages, table, layout, start, kind, rows=None, *, blocks=1, status=None):
    """down_project with the latents written straight into beacon pages:
    row i of request b becomes beacon `start + i` of that request (its K
    latent when kind == 'k', V latent when 'v'), at the BeaconPageLayout
    position table[b, (start + i) // slots].  pages [num_pages, >= page
    elements] bf16, table [B, T] int64 under torch's indexing rules.  A row
    mapping outside the table or pool is not written; `status` as
    beacon_pages."""
    _need_device(x, weight, rows, pages, table)
    _need_bf16(x, weight, pages)
    if kind not in ('k', 'v'):
        raise ValueError("kind must be 'k' or 'v'")
    if x.dim() != 3 or weight.dim() != 2 or weight.shape[1] != x.shape[2]:
        raise ValueError('x must be [B, L, K] and weight [N, K]')
    if pages.dim() != 2 or pages.stride(1) != 1 or pages.shape[1] < layout.page_elements:
        raise ValueError('pages must be [num_pages, page_elements] with contiguous rows')
    if table.dtype != torch.int64 or table.dim() != 2 or table.shape[0] != x.shape[0]:
        raise ValueError('table must be int64 [B, T]')
    N = weight.shape[0]
    if N != (layout.key_rank if kind == 'k' else layout.value_rank):
        raise ValueError('weight rows differ from the layout rank')
    x = _last_contiguous(x)
    weight = weight.contiguous()
    table = table if table.stride(1) == 1 else table.contiguous()
    B, L, K = x.shape
    if rows is not None:
        rows = rows.to(dtype=torch.long).contiguous()
    n = L if rows is None else rows.numel()
    a = _lib.DownProjectArgs(_ptr(x), x.stride(0), x.stride(1), _ptr(rows), n, L, _ptr(weight),
                             _ptr(pages), 0, 0, B, K, N, int(blocks))
    status, owned = _status_word(status, pages.device)
    dst = _lib.PageRows(_ptr(pages), pages.shape[0], pages.stride(0), _ptr(table), table.stride(0), table.shape[1],
                        layout.slots, layout.sink_elements, layout.width, 0 if kind == 'k' else layout.key_rank,
                        int(start), _ptr(status))
    nbytes = lib().slimkv_down_project_workspace(ctypes.byref(a))
    if nbytes == 0:
        check(-1)
    ws = _workspace(nbytes, x.device)
    check(lib().slimkv_down_project_to_pages(ctypes.byref(a), ctypes.byref(dst), _ptr(ws), nbytes,
                                             _lib.stream_handle(x.device)))
    if owned:
        check_status(status)
    return pages


def prepare_latent_bases(up_k, kv_heads):
    """Per-head transposed K bases [Hkv, Rk/Hkv, D] of a block-diagonal up_k
    [Hkv*D, Rk], made once per weight version and cached on the tensor."""
    _need_device(up_k)
    _need_bf16(up_k)
    key = (up_k._version, kv_heads, up_k.data_ptr())
    cached = getattr(up_k, '_slimkv_bases', None)
    if cached is not None and cached[0] == key:
        return cached[1]
    out_features, rank = up_k.shape
    if rank % kv_heads or out_features % kv_heads:
        raise ValueError('bases must split evenly across KV heads')
    w = up_k.contiguous()
    bases = torch.empty(kv_heads, rank // kv_heads, out_features // kv_heads, dtype=BF16, device=up_k.device)
    check(lib().slimkv_prepare_latent_bases(_ptr(w), kv_heads, out_features // kv_heads, rank, _ptr(bases),
                                            _lib.stream_handle(up_k.device)))
    up_k._slimkv_bases = (key, bases)
    return bases


def _latent_rows(lat_k, lat_v, Rk, Rv):
    lat_k, lat_v = _last_contiguous(lat_k), _last_contiguous(lat_v)
    if lat_k.dim() == 4:
        lat_k, lat_v = lat_k.squeeze(2), lat_v.squeeze(2)
    if lat_k.shape[-1] != Rk or lat_v.shape[-1] != Rv:
        raise ValueError('latent widths differ from the up-projection ranks')
    return lat_k, lat_v


def _latent_args(q, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale, up_k_bias, up_v_bias, block_diagonal,
                 lat_causal, q_positions, cos, sin, raw_lengths, lat_lengths, raw_splits, lat_splits, out, lse,
                 prepared_bases=True, lat_rows=None, lat_k2=None, lat_v2=None, raw_shape=None):
    """raw_shape = (raw rows, KV heads) when the raw rows are read through raw
    pages (raw_k / raw_v None)."""
    _need_device(q, raw_k, raw_v, lat_k, lat_v, lat_k2, lat_v2, up_k, up_v)
    _need_bf16(q, raw_k, raw_v, lat_k, lat_v, lat_k2, lat_v2, up_k, up_v, up_k_bias, up_v_bias)
    B, Lq, Hq, D = q.shape
    Nr, Hkv = raw_shape if raw_k is None else (raw_k.shape[1], raw_k.shape[2])
    Rk, Rv = up_k.shape[1], up_v.shape[1]
    # a second latent segment joins the first one's rows; an empty segment drops out
    if lat_k2 is not None and lat_k2.shape[1] == 0:
        lat_k2 = lat_v2 = None
    if lat_k2 is not None and (lat_k is None or lat_k.shape[1] == 0):
        lat_k, lat_v, lat_k2, lat_v2 = lat_k2, lat_v2, None, None
    Nl = (0 if lat_rows is None else int(lat_rows)) if lat_k is None else lat_k.shape[1]
    split = 0
    q = _last_contiguous(q)
    if raw_k is not None:
        raw_k, raw_v = _last_contiguous(raw_k), _last_contiguous(raw_v)
    if lat_k is not None:
        lat_k, lat_v = _latent_rows(lat_k, lat_v, Rk, Rv)
    if lat_k2 is not None:
        lat_k2, lat_v2 = _latent_rows(lat_k2, lat_v2, Rk, Rv)
        if lat_k2.shape[0] != lat_k.shape[0]:
            raise ValueError('latent segments differ in batch size')
        split, Nl = Nl, Nl + lat_k2.shape[1]
    up_k, up_v = up_k.contiguous(), up_v.contiguous()
    if out is None:
        out = torch.empty(B, Lq, Hq, D, dtype=BF16, device=q.device)
    if lse is None:
        lse = torch.empty(B, Hq, Lq, dtype=torch.float32, device=q.device)
    if cos is not None:
        if cos.dtype != torch.float32 or sin.dtype != torch.float32:
            raise ValueError('RoPE tables must be fp32')
        if q_positions is None:
            # tables already taken at the query positions (query_rope_rows)
            cos, sin = cos.reshape(-1, D), sin.reshape(-1, D)
            if cos.shape[0] < B * Lq or sin.shape != cos.shape:
                raise ValueError('RoPE rows at the query positions must cover [B, Lq, D]')
        else:
            q_positions = q_positions.to(torch.int64)
            if q_positions.stride(-1) != 1:
                q_positions = q_positions.contiguous()
        cos, sin = cos.contiguous(), sin.contiguous()
    bases = None
    if prepared_bases and block_diagonal and Nl > 0 and Rk % Hkv == 0 \
            and (Rk // Hkv) % 16 == 0 and D == 128:
        bases = prepare_latent_bases(up_k, Hkv)
    a = _lib.LatentDecodeArgs(
        _ptr(q), *q.stride()[:3],
        _ptr(q_positions), 0 if q_positions is None else q_positions.stride(0),
        _ptr(cos), _ptr(sin), 0 if cos is None else cos.shape[0],
        _ptr(raw_k), *(raw_k.stride()[:3] if raw_k is not None else (0, 0, 0)),
        _ptr(raw_v), *(raw_v.stride()[:3] if raw_v is not None else (0, 0, 0)),
        _ptr(raw_lengths), Nr,
        _ptr(lat_k), *(lat_k.stride()[:2] if lat_k is not None else (0, 0)),
        _ptr(lat_v), *(lat_v.stride()[:2] if lat_v is not None else (0, 0)),
        _ptr(lat_lengths), Nl, int(bool(lat_causal)), int(bool(block_diagonal)),
        _ptr(up_k), _ptr(up_k_bias), _ptr(up_v), _ptr(up_v_bias),
        B, Lq, Hq, Hkv, D, Rk, Rv, float(scale),
        _ptr(out), *out.stride()[:3], _ptr(lse), int(raw_splits), int(lat_splits), _ptr(bases),
        _ptr(lat_k2), *(lat_k2.stride()[:2] if lat_k2 is not None else (0, 0)),
        _ptr(lat_v2), *(lat_v2.stride()[:2] if lat_v2 is not None else (0, 0)), split)
    keep = (q, raw_k, raw_v, lat_k, lat_v, lat_k2, lat_v2, up_k, up_v, cos, sin, q_positions, bases)
    return a, out, lse, keep


def query_rope_rows(cos, sin, q_positions):
    """cos/sin rows at the query positions [B, Lq] -> ([B*Lq, D], [B*Lq, D]).

    Every layer of a decode step rotates its queries at the same positions, so
    the rows are gathered once per step (as a model's rotary embedding returns
    them) and passed to each layer's latent_decode with q_positions=None; the
    rotation is then the same, without the position lookup in every layer.
    Positions are clamped into the tables like the kernels clamp them."""
    _need_device(cos, sin, q_positions)
    idx = q_positions.reshape(-1).to(torch.int64).clamp(0, cos.shape[0] - 1)
    return cos.index_select(0, idx), sin.index_select(0, idx)


def latent_decode(q, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale, *, up_k_bias=None, up_v_bias=None,
                  block_diagonal=False, lat_causal=False, q_positions=None, cos=None, sin=None,
                  raw_lengths=None, lat_lengths=None, raw_splits=0, lat_splits=0, out=None, lse=None,
                  workspace=None, prepared_bases=True, stages=_lib.STAGE_ALL, lat_k2=None, lat_v2=None):
    """Fused latent beacon decode for one layer.

    q [B,Lq,Hq,D] (rotated in-kernel at q_positions when cos/sin are given;
    without q_positions, cos/sin are the rows at the query positions, see
    query_rope_rows),
    raw_k/raw_v [B,Nr,Hkv,D] with RoPE'd K, lat_k [B,Nl,Rk], lat_v [B,Nl,Rv],
    up_k [Hkv*D,Rk], up_v [Hkv*D,Rv].  Returns (out [B,Lq,Hq,D] bf16, lse [B,Hq,Lq]).
    A caller-provided `workspace` (uint8, at least latent_decode_workspace_bytes)
    makes the call allocation-free, e.g. under HIP graph capture.  With
    block-diagonal bases the query absorption runs on MFMA from per-head bases
    prepared once per weight (`prepared_bases`, the default).  `stages`
    (a mask of _lib.STAGE_*) runs part of the call; the stages of one decode
    hand over through `workspace`, which is then required.  lat_k2 / lat_v2
    [B, N2, R*] hold latent rows that follow lat_k / lat_v's (a history and
    the current window read where they lie, without joining them).
    """
    a, out, lse, keep = _latent_args(q, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale, up_k_bias, up_v_bias,
                                     block_diagonal, lat_causal, q_positions, cos, sin, raw_lengths,
                                     lat_lengths, raw_splits, lat_splits, out, lse, prepared_bases,
                                     lat_k2=lat_k2, lat_v2=lat_v2)
    nbytes = lib().slimkv_latent_decode_workspace(ctypes.byref(a))
    if nbytes == 0:
        check(-1)
    workspace = _stage_workspace(workspace, nbytes, stages, q.device)
    if stages == _lib.STAGE_ALL:
        check(lib().slimkv_latent_decode(ctypes.byref(a), _ptr(workspace), nbytes, _lib.stream_handle(q.device)))
    else:
        check(lib().slimkv_latent_decode_stages(ctypes.byref(a), int(stages), _ptr(workspace), nbytes,
                                                _lib.stream_handle(q.device)))
    del keep
    return out, lse


def _stage_workspace(workspace, nbytes, stages, device):
    if workspace is not None and workspace.numel() >= nbytes:
        return workspace
    if stages != _lib.STAGE_ALL:
        raise ValueError('a partial-stage call needs the workspace its other stages use')
    return _workspace(nbytes, device)


def paged_latent_decode(q, raw_k, raw_v, pages, table, lat_lengths, lat_keys, layout, up_k, up_v, scale, *,
                        rows_total=0, up_k_bias=None, up_v_bias=None, block_diagonal=False, lat_causal=False,
                        q_positions=None, cos=None, sin=None, raw_lengths=None, raw_splits=0, lat_splits=0,
                        out=None, lse=None, workspace=None, stages=_lib.STAGE_ALL, status=None,
                        raw_pages=None, raw_tables=None, raw_keys=None):
    """latent_decode with the beacon rows read straight out of beacon pages.

    pages [num_pages, layout.page_elements] bf16 in BeaconPageLayout format;
    table [B, >= ceil(lat_keys / slots)] int64 page ids; lat_lengths [B] int32
    beacons per sequence (<= lat_keys).  rows_total = sum of lat_lengths when
    known on the host (sizes the key splits only).  Same result as gathering
    the rows (BeaconPages.read_batch) and calling latent_decode.  Table
    entries follow torch's indexing rules; an entry outside the pool that a
    beacon needs raises IndexError after the call (one host synchronisation)
    unless the caller passes its own device int32 `status` word (graph
    capture, serving loops) and checks it with check_status.

    raw_pages [blocks, block, 2, Hkv, D] (RawPages' pages) with raw_tables
    [B, cols] int64 and raw_lengths [B] int32: the raw rows are read through
    the raw block table as well (raw_k / raw_v None; raw_keys = the largest
    raw row count, default cols * block).  Same result as RawPages.read_batch
    into dense rows followed by this call.
    """
    _need_device(pages, table, lat_lengths, raw_pages, raw_tables)
    _need_bf16(pages)
    if up_k.shape[1] != layout.key_rank or up_v.shape[1] != layout.value_rank:
        raise ValueError('page layout ranks differ from the up-projection ranks')
    if pages.dim() != 2 or pages.stride(1) != 1 or pages.shape[1] < layout.page_elements:
        raise ValueError('pages must be [num_pages, page_elements] with contiguous rows')
    if table.dtype != torch.int64 or table.dim() != 2 or lat_lengths.dtype != torch.int32:
        raise ValueError('table must be int64 [B, pages], lat_lengths int32 [B]')
    table = table if table.stride(1) == 1 else table.contiguous()
    lat_lengths = lat_lengths.contiguous()
    raw_fields = (None, 0, 0, 0, 0, 0, 0, None, 0, 0)
    raw_shape = None
    if raw_pages is not None:
        _need_bf16(raw_pages)
        if raw_pages.dim() != 5 or raw_pages.shape[2] != 2 or raw_pages.stride(4) != 1:
            raise ValueError('raw pages must be [blocks, block, 2, Hkv, D] with contiguous rows')
        if raw_tables is None or raw_tables.dtype != torch.int64 or raw_tables.dim() != 2 or raw_lengths is None:
            raise ValueError('raw pages need int64 raw_tables [B, cols] and raw_lengths')
        raw_tables = raw_tables if raw_tables.stride(1) == 1 else raw_tables.contiguous()
        block = raw_pages.shape[1]
        raw_keys = raw_tables.shape[1] * block if raw_keys is None else int(raw_keys)
        raw_shape = (raw_keys, raw_pages.shape[3])
        st = raw_pages.stride()
        raw_fields = (_ptr(raw_pages), raw_pages.shape[0], block, st[0], st[1], st[2], st[3], _ptr(raw_tables),
                      raw_tables.stride(0), raw_tables.shape[1])
        raw_k = raw_v = None
    base, out, lse, keep = _latent_args(q, raw_k, raw_v, None, None, up_k, up_v, scale, up_k_bias, up_v_bias,
                                        block_diagonal, lat_causal, q_positions, cos, sin, raw_lengths,
                                        lat_lengths, raw_splits, lat_splits, out, lse, True, lat_rows=lat_keys,
                                        raw_shape=raw_shape)
    status, owned = _status_word(status, pages.device)
    a = _lib.PagedLatentDecodeArgs(base, _ptr(pages), pages.shape[0], pages.stride(0), _ptr(table), table.stride(0),
                                   table.shape[1], layout.slots, layout.sink_elements, int(rows_total), _ptr(status),
                                   *raw_fields)
    nbytes = lib().slimkv_paged_latent_decode_workspace(ctypes.byref(a))
    if nbytes == 0:
        check(-1)
    workspace = _stage_workspace(workspace, nbytes, stages, q.device)
    if stages == _lib.STAGE_ALL:
        check(lib().slimkv_paged_latent_decode(ctypes.byref(a), _ptr(workspace), nbytes,
                                               _lib.stream_handle(q.device)))
    else:
        check(lib().slimkv_paged_latent_decode_stages(ctypes.byref(a), int(stages), _ptr(workspace), nbytes,
                                                      _lib.stream_handle(q.device)))
    if owned and stages & _lib.STAGE_ATTEND:
        check_status(status)
    del keep
    return out, lse


def latent_decode_workspace_bytes(q, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale=1.0, **kw):
    """Workspace bytes latent_decode needs for these tensors (same keywords)."""
    names = ('up_k_bias', 'up_v_bias', 'block_diagonal', 'lat_causal', 'q_positions', 'cos', 'sin',
             'raw_lengths', 'lat_lengths', 'raw_splits', 'lat_splits', 'out', 'lse')
    defaults = dict(up_k_bias=None, up_v_bias=None, block_diagonal=False, lat_causal=False, q_positions=None,
                    cos=None, sin=None, raw_lengths=None, lat_lengths=None, raw_splits=0, lat_splits=0,
                    out=None, lse=None)
    defaults.update({k: v for k, v in kw.items() if k in names})
    a, _, _, keep = _latent_args(q, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale,
                                 *(defaults[n] for n in names))
    nbytes = lib().slimkv_latent_decode_workspace(ctypes.byref(a))
    if nbytes == 0:
        check(-1)
    del keep
    return nbytes


def reconstruct(latent, weight, bias=None, *, kv_heads, out=None, dst_rows=None, positions=None, cos=None,
                sin=None, block_diagonal=False):
    """Up-project latent rows [B, n, R] with an nn.Linear weight [Hkv*D, R] into
    out [B, rows, Hkv, D] (any 4-D view with a contiguous last dim), optionally
    scattered to dst_rows and RoPE'd at positions [B, n]."""
    a, out, keep = _reconstruct_args(latent, weight, bias, kv_heads, out, dst_rows, positions, cos, sin,
                                     block_diagonal)
    check(lib().slimkv_reconstruct(ctypes.byref(a), _lib.stream_handle(keep[0].device)))
    return out


def reconstruct_pair(first, second):
    """Two reconstructions in one launch where the library can (both on its
    streaming kernel at one latent width, as the K and V rebuild of a
    window's beacon rows are), the same bits as two reconstruct calls.
    `first` / `second`: dicts of reconstruct's arguments.  Returns the two
    outputs."""
    a, out_a, keep_a = _reconstruct_args(**_recon_kwargs(first))
    b, out_b, keep_b = _reconstruct_args(**_recon_kwargs(second))
    if keep_a[0].device != keep_b[0].device:
        raise ValueError('both reconstructions must be on one device')
    check(lib().slimkv_reconstruct_pair(ctypes.byref(a), ctypes.byref(b), _lib.stream_handle(keep_a[0].device)))
    return out_a, out_b


def _recon_kwargs(kw):
    names = ('latent', 'weight', 'bias', 'kv_heads', 'out', 'dst_rows', 'positions', 'cos', 'sin', 'block_diagonal')
    unknown = set(kw) - set(names)
    if unknown:
        raise TypeError(f'unknown reconstruct arguments {sorted(unknown)}')
    defaults = dict(bias=None, out=None, dst_rows=None, positions=None, cos=None, sin=None, block_diagonal=False)
    return {n: kw.get(n, defaults.get(n)) for n in names}


def _reconstruct_args(latent, weight, bias, kv_heads, out, dst_rows, positions, cos, sin, block_diagonal):
    """The slimkv_reconstruct_args of one reconstruction, its output, and the
    tensors the arguments point into (kept alive until the launch)."""
    _need_device(latent, weight, bias, out)
    _need_bf16(latent, weight, bias, out)
    latent = _last_contiguous(latent)
    weight = weight.contiguous()
    B, n, R = latent.shape
    D = weight.shape[0] // kv_heads
    if out is None:
        out = torch.empty(B, n, kv_heads, D, dtype=BF16, device=latent.device)
    if dst_rows is not None:
        dst_rows = dst_rows.to(device=latent.device, dtype=torch.int64).contiguous()
    if positions is not None:
        positions = positions.to(torch.int64)
        positions = positions if positions.stride(-1) == 1 else positions.contiguous()
    a = _lib.ReconstructArgs(
        _ptr(latent), latent.stride(0), latent.stride(1), _ptr(weight), _ptr(bias),
        _ptr(out), out.stride(0), out.stride(1), out.stride(2), _ptr(dst_rows),
        _ptr(cos), _ptr(sin), 0 if cos is None else cos.shape[0],
        _ptr(positions), 0 if positions is None else positions.stride(0),
        B, n, R, kv_heads, D, int(bool(block_diagonal)))
    return a, out, (latent, weight, bias, out, dst_rows, positions, cos, sin)


def recon_decode(q, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale, *, beacon_positions=None, up_k_bias=None,
                 up_v_bias=None, block_diagonal=False, lat_causal=False, q_positions=None, cos=None, sin=None,
                 raw_lengths=None, lat_lengths=None, raw_splits=0, lat_splits=0, out=None, lse=None, workspace=None,
                 stages=_lib.STAGE_ALL, reference_rounding=False):
    """Reconstruction decode: rebuild beacon K (RoPE'd at beacon_positions
    [B, Nl] when given) and V, then attend over [beacons ; raw rows].
    `stages` as latent_decode.  On the fused route (block-diagonal bases)
    rotated beacon keys are rebuilt in fp32 and rounded once, unless
    reference_rounding asks for the reference's bf16 steps (the bits
    ReconstructionCache.materialize writes, modeling_llama.py:1405-1483)."""
    base, out, lse, keep = _latent_args(q, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale, up_k_bias, up_v_bias,
                                        block_diagonal, lat_causal, q_positions, cos, sin, raw_lengths,
                                        lat_lengths, raw_splits, lat_splits, out, lse, prepared_bases=False)
    pairs = None
    if beacon_positions is not None:
        beacon_positions = beacon_positions.to(torch.int64)
        beacon_positions = beacon_positions if beacon_positions.stride(-1) == 1 else beacon_positions.contiguous()
        if cos is None:
            raise ValueError('beacon RoPE needs the cos/sin tables')
        pairs, repeats = prepare_rope_pairs(cos, sin)
    a = _lib.ReconDecodeArgs(base, _ptr(beacon_positions),
                             0 if beacon_positions is None else beacon_positions.stride(0), _ptr(pairs),
                             int(pairs is not None and repeats), int(not reference_rounding))
    nbytes = lib().slimkv_recon_decode_workspace(ctypes.byref(a))
    if nbytes == 0:
        check(-1)
    workspace = _stage_workspace(workspace, nbytes, stages, q.device)
    if stages == _lib.STAGE_ALL:
        check(lib().slimkv_recon_decode(ctypes.byref(a), _ptr(workspace), nbytes, _lib.stream_handle(q.device)))
    else:
        check(lib().slimkv_recon_decode_stages(ctypes.byref(a), int(stages), _ptr(workspace), nbytes,
                                               _lib.stream_handle(q.device)))
    del keep
    return out, lse


def prepare_rope_pairs(cos, sin):
    """((bf16 cos | bf16 sin << 16) as int32 [rows, dim], repeats) built once
    per table pair and cached on `cos` (keyed by both tables' versions and
    pointers).  repeats: every row is its first half twice (rotate-half
    tables), checked once here (one host synchronisation per table)."""
    _need_device(cos, sin)
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape != sin.shape or cos.dim() != 2:
        raise ValueError('RoPE tables must be fp32 [rows, dim] of equal shape')
    key = (cos._version, sin._version, cos.data_ptr(), sin.data_ptr())
    cached = getattr(cos, '_slimkv_pairs', None)
    if cached is not None and cached[0] == key:
        return cached[1], cached[2]
    c, s_ = cos.contiguous(), sin.contiguous()
    out = torch.empty(cos.shape, dtype=torch.int32, device=cos.device)
    check(lib().slimkv_prepare_rope_pairs(_ptr(c), _ptr(s_), cos.shape[0], cos.shape[1], _ptr(out),
                                          _lib.stream_handle(cos.device)))
    half = cos.shape[1] // 2
    repeats = bool(cos.shape[1] % 2 == 0 and torch.equal(out[:, :half], out[:, half:]))
    cos._slimkv_pairs = (key, out, repeats)
    return out, repeats


def rope_decode(q, k, cos, sin, query_positions, raw_indices, sink, history):
    """q [B,Hq,Lq,D], k [B,Hk,Nk,D] (BHSD); returns new contiguous (oq, ok)."""
    _need_device(q, k, cos, sin, query_positions)
    _need_bf16(q, k)
    q, k = _last_contiguous(q), _last_contiguous(k)
    oq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    ok = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    pos = query_positions if query_positions.dtype == torch.int64 else query_positions.long()
    if pos.stride(-1) != 1:
        pos = pos.contiguous()
    idx = None
    if raw_indices is not None:
        idx = raw_indices.to(device=q.device, dtype=torch.int64).contiguous()
    a = _lib.RopeDecodeArgs(
        _ptr(q), q.stride(0), q.stride(1), q.stride(2),
        _ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _ptr(oq), _ptr(ok), _ptr(cos), _ptr(sin), cos.shape[0],
        _ptr(pos), pos.stride(0), _ptr(idx), 0 if idx is None else idx.numel(),
        q.shape[0], q.shape[1], k.shape[1], q.shape[2], k.shape[2], q.shape[3], int(sink), int(history))
    check(lib().slimkv_rope_decode(ctypes.byref(a), _lib.stream_handle(q.device)))
    return oq, ok


def linear_rows(x, weight, bias=None, out=None):
    """Projection of a decode step's rows: x [..., K] (at most 4 rows) ->
    out [..., N] = x W^T (+ bias), W the nn.Linear weight [N, K] bf16
    (N a multiple of 128), fp32 accumulation, one bf16 rounding."""
    _need_device(x, weight, bias)
    _need_bf16(x, weight)
    N, K = weight.shape
    if x.shape[-1] != K or weight.stride(-1) != 1 or weight.stride(0) != K:
        raise ValueError('x [..., K] against a contiguous weight [N, K] required')
    rows = x.reshape(-1, K)
    if rows.stride(-1) != 1:
        rows = rows.contiguous()
    if out is None:
        out = torch.empty(*x.shape[:-1], N, dtype=BF16, device=x.device)
    flat = out.view(-1, N)
    if bias is not None and (bias.dtype != BF16 or not bias.is_contiguous() or bias.numel() != N):
        raise ValueError('bias must be a contiguous bf16 [N]')
    a = _lib.LinearRowsArgs(_ptr(rows), rows.stride(0), _ptr(weight), _ptr(bias), _ptr(flat), flat.stride(0),
                            rows.shape[0], N, K)
    check(lib().slimkv_linear_rows(ctypes.byref(a), _lib.stream_handle(x.device)))
    return out


def _check_qkv_shapes(x, weight, bias, heads, kv_heads, positions, q_out):
    """Shapes slimkv_decode_qkv indexes without bounds: x [B, K] with 1 <= B <= 4,
    a contiguous weight [(heads + 2 kv_heads) * 128, K], a bias of that many
    elements, at least B positions, q_out [B, heads * 128]."""
    if heads <= 0 or kv_heads <= 0 or heads % kv_heads:
        raise ValueError('heads must be a positive multiple of kv_heads')
    if x.dim() != 2 or not 1 <= x.shape[0] <= 4:
        raise ValueError('x must be [B, K] with 1 <= B <= 4 rows')
    B, K = x.shape
    N = (heads + 2 * kv_heads) * 128
    if weight.dim() != 2 or tuple(weight.shape) != (N, K) or not weight.is_contiguous():
        raise ValueError(f'weight must be a contiguous [(heads + 2 kv_heads) * 128, K] = [{N}, {K}], '
                         f'found {list(weight.shape)}')
    if bias is not None and (bias.numel() != N or not bias.is_contiguous() or bias.dtype != BF16):
        raise ValueError(f'bias must be a contiguous bf16 [{N}]')
    if positions.dim() > 1 or positions.numel() < B:
        raise ValueError(f'positions must be a 1-D tensor of at least B = {B} entries')
    if q_out is not None and (tuple(q_out.shape) != (B, heads * 128) or q_out.stride(-1) != 1
                              or q_out.dtype != BF16):
        raise ValueError(f'q_out must be bf16 [{B}, {heads * 128}] with unit last stride')


def decode_qkv(x, weight, bias, heads, kv_heads, cos, sin, positions, raw_k, raw_v, slot_index, plain_k=None,
               q_out=None, status=None):
    """The new token's q/k/v projection, key RoPE and raw-cache appends in one
    launch.  x [B, K] (B <= 4 rows), weight = cat([W_q, W_k, W_v]) [(Hq + 2 Hkv)
    * 128, K] (bias likewise or None), positions [B] int64, caches
    [B, capacity, Hkv, 128] (rotated K, V and optionally unrotated K) written at
    slot = slot_index[0] (device int64).  Returns q [B, Hq * 128] unrotated.
    A slot outside [0, capacity) writes no cache row: without a caller `status`
    word (device int32) that raises IndexError here (one host synchronisation,
    refused under graph capture); with one, SLIMKV_STATUS_BAD_SLOT is left in
    it (the reference's index_copy_ raises IndexError)."""
    _check_qkv_shapes(x, weight, bias, heads, kv_heads, positions, q_out)
    _need_device(x, weight, bias, cos, sin, positions, raw_k, raw_v, slot_index, plain_k, q_out)
    _need_bf16(x, weight, raw_k, raw_v)
    B, K = x.shape
    if x.stride(-1) != 1:
        x = x.contiguous()
    caches = [c for c in (raw_k, raw_v, plain_k) if c is not None]
    if any(c.stride() != raw_k.stride() or c.shape != raw_k.shape for c in caches) or raw_k.stride(-1) != 1 \
            or raw_k.stride(2) != 128 or raw_k.shape[2] != kv_heads or raw_k.shape[0] != B:
        raise ValueError('the caches must share shape [B, capacity, Hkv, 128] and strides')
    if slot_index.numel() < 1:
        raise ValueError('slot_index must hold the slot')
    if q_out is None:
        q_out = torch.empty(B, heads * 128, dtype=BF16, device=x.device)
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or not cos.is_contiguous() or \
            not sin.is_contiguous() or cos.shape != sin.shape or cos.shape[-1] != 128:
        raise ValueError('RoPE tables must be contiguous fp32 [rows, 128]')
    if status is None and torch.cuda.is_current_stream_capturing():
        raise ValueError('decode_qkv under graph capture needs a caller status word')
    status, owned = _status_word(status, x.device)
    pos = positions.to(torch.int64)
    slot = slot_index.to(torch.int64)
    a = _lib.DecodeQKVArgs(_ptr(x), x.stride(0), _ptr(weight), _ptr(bias), _ptr(q_out), q_out.stride(0),
                           _ptr(raw_k), _ptr(plain_k), _ptr(raw_v), raw_k.stride(0), raw_k.stride(1), _ptr(slot),
                           _ptr(cos), _ptr(sin), cos.shape[0], _ptr(pos), pos.stride(0) if pos.dim() else 1,
                           B, K, heads, kv_heads, 128, raw_k.shape[1], _ptr(status))
    check(lib().slimkv_decode_qkv(ctypes.byref(a), _lib.stream_handle(x.device)))
    if owned:
        check_status(status)
    return q_out


def prefill_rope(q, k, cos, sin, positions, roles, sink, out_q=None, out_k=None):
    """q [B,Hq,Lq,D], k [B,Hk,Nk,D]; outputs keep the input strides
    (empty_like) unless the caller passes them (out_q / out_k of the inputs'
    shapes, rows 16-byte aligned, not overlapping the inputs: a row's
    rotate-half partner is read by another thread)."""
    _need_device(q, k, cos, sin, positions, roles, out_q, out_k)
    _need_bf16(q, k, out_q, out_k)
    oq = torch.empty_like(q) if out_q is None else out_q
    ok = torch.empty_like(k) if out_k is None else out_k
    if oq.shape != q.shape or ok.shape != k.shape or oq.stride(-1) != 1 or ok.stride(-1) != 1:
        raise ValueError('RoPE outputs must have the shapes of q and k with contiguous rows')
    pos = positions if positions.stride(-1) == 1 else positions.contiguous()
    roles = roles.to(device=q.device, dtype=torch.int64).contiguous()
    a = _lib.PrefillRopeArgs(
        _ptr(q), *q.stride()[:3], _ptr(k), *k.stride()[:3],
        _ptr(oq), *oq.stride()[:3], _ptr(ok), *ok.stride()[:3],
        _ptr(cos), _ptr(sin), cos.shape[0], _ptr(pos), pos.stride(0),
        _ptr(roles), roles.numel(),
        q.shape[0], q.shape[1], k.shape[1], q.shape[2], k.shape[2], q.shape[3], int(sink))
    check(lib().slimkv_prefill_rope(ctypes.byref(a), _lib.stream_handle(q.device)))
    return oq, ok


def rope_keys(k, cos, sin, positions, roles, sink, out_k=None, v=None, out_v=None):
    """The key half of prefill_rope: k [B,Hk,Nk,D] rotated (beacon keys
    copied unchanged) into out_k (default empty_like); for an attention that
    rotates its own queries (prefill_attention with q_positions).  With v
    and out_v (both of k's shape) the value rows are copied into out_v in the
    same launch."""
    _need_device(k, cos, sin, positions, roles, out_k, v, out_v)
    _need_bf16(k, out_k, v, out_v)
    ok = torch.empty_like(k) if out_k is None else out_k
    if ok.shape != k.shape or ok.stride(-1) != 1:
        raise ValueError('the RoPE output must have the shape of k with contiguous rows')
    if (v is None) != (out_v is None):
        raise ValueError('the value rows need both v and out_v')
    if v is not None and (v.shape != k.shape or out_v.shape != k.shape or v.stride(-1) != 1 or
                          out_v.stride(-1) != 1):
        raise ValueError('v and out_v must have the shape of k with contiguous rows')
    pos = positions if positions.stride(-1) == 1 else positions.contiguous()
    roles = roles.to(device=k.device, dtype=torch.int64).contiguous()
    B, Hk, Nk, D = k.shape
    a = _lib.PrefillRopeArgs(
        None, 0, 0, 0, _ptr(k), *k.stride()[:3],
        None, 0, 0, 0, _ptr(ok), *ok.stride()[:3],
        _ptr(cos), _ptr(sin), cos.shape[0], _ptr(pos), pos.stride(0),
        _ptr(roles), roles.numel(),
        B, Hk, Hk, 0, Nk, D, int(sink),
        _ptr(v), *(v.stride()[:3] if v is not None else (0, 0, 0)),
        _ptr(out_v), *(out_v.stride()[:3] if out_v is not None else (0, 0, 0)))
    check(lib().slimkv_prefill_rope(ctypes.byref(a), _lib.stream_handle(k.device)))
    return ok


_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16, torch.float32: _lib.DTYPE_F32}


def _dtype_code(*tensors):
    dt = tensors[0].dtype
    if dt not in _DTYPES or any(t.dtype != dt for t in tensors):
        raise ValueError(f'expected one of bfloat16, float16, float32 for every tensor, found '
                         f'{[t.dtype for t in tensors]}')
    return _DTYPES[dt]


def merge(raw, raw_lse, latent, latent_lse):
    """raw/latent [B,H,L,D] (bf16, fp16 or fp32), LSEs [B,H,L] -> contiguous
    [B,H,L,D] in the branches' dtype, merged in fp32 and rounded once."""
    _need_device(raw, latent, raw_lse, latent_lse)
    code = _dtype_code(raw, latent)
    raw, latent = _last_contiguous(raw), _last_contiguous(latent)
    raw_lse, latent_lse = raw_lse.float(), latent_lse.float()
    out = torch.empty(raw.shape, dtype=raw.dtype, device=raw.device)
    a = _lib.MergeArgs(
        _ptr(raw), *raw.stride()[:3], _ptr(latent), *latent.stride()[:3],
        _ptr(raw_lse), *raw_lse.stride(), _ptr(latent_lse), *latent_lse.stride(),
        _ptr(out), *raw.shape)
    vector = (code == _lib.DTYPE_BF16 and raw.shape[-1] % 8 == 0
              and all(x % 8 == 0 for x in (*raw.stride()[:3], *latent.stride()[:3]))
              and all(t.data_ptr() % 16 == 0 for t in (raw, latent, out)))
    if vector:
        check(lib().slimkv_merge(ctypes.byref(a), _lib.stream_handle(raw.device)))
    else:
        check(lib().slimkv_merge_typed(ctypes.byref(a), code, _lib.stream_handle(raw.device)))
    return out


def eager_attention(q, k, v, scale, causal=False):
    """fp32 attention (latent_decode.eager_forward arithmetic) for bf16, fp16 or
    fp32 BSHD tensors: q [B,Lq,H,R], k [B,N,Hk,R], v [B,N,Hk,Rv] ->
    (out [B,Lq,H,Rv] in q's dtype, lse [B,H,Lq] fp32)."""
    _need_device(q, k, v)
    code = _dtype_code(q, k, v)
    q, k, v = (_last_contiguous(x) for x in (q, k, v))
    B, Lq, H, R = q.shape
    N, Hk = k.shape[1], k.shape[2]
    out = torch.empty(B, Lq, H, v.shape[-1], dtype=q.dtype, device=q.device)
    lse = torch.empty(B, H, Lq, dtype=torch.float32, device=q.device)
    scores = torch.empty(max(B * H * Lq * N, 1), dtype=torch.float32, device=q.device)
    a = _lib.EagerAttentionArgs(
        _ptr(q), *q.stride()[:3], _ptr(k), *k.stride()[:3], _ptr(v), *v.stride()[:3],
        _ptr(out), *out.stride()[:3], _ptr(lse), _ptr(scores),
        B, Lq, H, Hk, N, R, v.shape[-1], float(scale), code, int(bool(causal)))
    check(lib().slimkv_eager_attention(ctypes.byref(a), _lib.stream_handle(q.device)))
    return out, lse


def default_scale(head_dim):
    return 1.0 / math.sqrt(head_dim)


def _status_word(status, device):
    """(status, owned): the caller's device int32 status word, or a fresh zeroed
    one that the call checks itself (one host synchronisation) when owned."""
    if status is not None:
        if status.dtype != torch.int32 or status.device != device or status.numel() < 1:
            raise ValueError('status must be a device int32 tensor on the tensors\' device')
        return status, False
    return torch.zeros(1, dtype=torch.int32, device=device), True


def check_status(status):
    """Raise IndexError when a kernel reported an index error in `status`: a
    block-table entry outside the pool (the reference's torch indexing raises
    IndexError, paged_cache.py:60-67) or a row outside its buffer: a decode
    cache slot past the caches (index_copy_, static_decode.py:156-163) or a
    paged request's raw set past the step's dense rows.  Synchronises the
    host."""
    code = int(status.reshape(-1)[0].item())
    if code == _lib.STATUS_BAD_SLOT:
        raise IndexError('cache slot outside the buffer (decode cache capacity or the dense raw rows)')
    if code != 0:
        raise IndexError('block table refers to a page outside the allocation')


def _table(table, device):
    """Block table as device int64 [B, T] (a 1-D table is one request)."""
    table = table.to(device=device, dtype=torch.long)
    if table.dim() == 1:
        table = table[None]
    if table.dim() != 2 or table.stride(1) != 1:
        table = table.reshape(table.shape[0], -1).contiguous()
    return table


def _lengths(lengths, batch, device):
    if lengths is None:
        return None
    lengths = lengths.to(device=device, dtype=torch.int32).contiguous()
    if lengths.shape != (batch,):
        raise ValueError('lengths must be [batch]')
    return lengths


def _starts(starts, batch, device):
    if starts is None:
        return None
    starts = starts.to(device=device, dtype=torch.int64).contiguous()
    if starts.shape != (batch,):
        raise ValueError('starts must be [batch]')
    return starts


def beacon_pages(pages, table, dense_k, dense_v, *, slots, key_rank, value_rank, sink_elements, start, count,
                 to_pages, lengths=None, status=None, starts=None):
    """Copy beacon latents between pages [num_pages, >=page_elements] and dense
    rows dense_k [B, count, key_rank], dense_v [B, count, value_rank]
    (slimkv/vllm_plugin/paged_cache.py:60-87).  table: [B, T] or [T] int64,
    entries under torch's indexing rules.  A row whose entry lies outside the
    pool moves nothing; without a caller `status` word that raises IndexError
    here (one host synchronisation), with one it is left in `status`.
    `starts` (device int64 [B], optional): request b's dense row r is beacon
    start + starts[b] + r (rows at or past lengths[b] are skipped)."""
    _need_device(pages, dense_k, dense_v)
    _need_bf16(pages, dense_k, dense_v)
    if pages.dim() != 2 or pages.stride(1) != 1:
        raise ValueError('pages must be [num_pages, features] with contiguous features')
    table = _table(table, pages.device)
    B = table.shape[0]
    for t, w in ((dense_k, key_rank), (dense_v, value_rank)):
        if t.dim() != 3 or t.shape != (B, count, w) or t.stride(2) != 1:
            raise ValueError(f'dense latents must be [{B}, {count}, {w}] with contiguous rows')
    lengths = _lengths(lengths, B, pages.device)
    starts = _starts(starts, B, pages.device)
    status, owned = _status_word(status, pages.device)
    a = _lib.BeaconPagesArgs(
        pages=_ptr(pages), num_pages=pages.shape[0], page_stride=pages.stride(0),
        table=_ptr(table), t_sb=table.stride(0), t_cols=table.shape[1],
        dense_k=_ptr(dense_k), dk_sb=dense_k.stride(0), dk_sn=dense_k.stride(1),
        dense_v=_ptr(dense_v), dv_sb=dense_v.stride(0), dv_sn=dense_v.stride(1),
        lengths=_ptr(lengths), batch=B, start=start, count=count, slots=slots, key_rank=key_rank,
        value_rank=value_rank, sink_elements=sink_elements, to_pages=int(bool(to_pages)), status=_ptr(status),
        starts=_ptr(starts))
    check(lib().slimkv_beacon_pages(ctypes.byref(a), _lib.stream_handle(pages.device)))
    if owned:
        check_status(status)


def paged_step_rows(raw_pages, raw_table, beacon_pages, beacon_table, new_k, new_v, window_start, raw_count,
                    positions, cos, sin, rows, sink, *, page_stride=None, flush=False, raw_write_end=None,
                    sink_update=None, out_k=None, out_v=None, status=None):
    """The dense raw set of one decode step for a batch of paged requests,
    K rotated: out_k / out_v [B, rows, Hkv, 128] with the sink (from the root
    beacon page beacon_table[:, 0]), the window rows (raw pages, positions
    window_start[b] + j for j < raw_count[b]) and the new token (new_k / new_v
    [B, Hkv, 128]) at rows 0, sink .. sink + raw_count - 1 and sink +
    raw_count; K rotated at positions [B, >= rows] (fp32 cos/sin).  With
    `flush`: flush_memory's writes afterwards (the new token into its raw page
    below raw_write_end, the sink replaced where sink_update).  Rows past a
    request's raw set are left unwritten; a request whose raw set (sink +
    raw_count + 1 rows) does not fit `rows` is an index error (the status
    word's bad-slot code).  Index errors as raw_pages."""
    _need_device(raw_pages, beacon_pages, new_k, new_v, window_start, raw_count, positions, cos, sin)
    _need_bf16(raw_pages, beacon_pages, new_k, new_v, out_k, out_v)
    if raw_pages.dim() != 5 or raw_pages.shape[2] != 2 or raw_pages.stride(4) != 1:
        raise ValueError('raw pages must be [blocks, block_size, 2, heads, dim] with contiguous dim')
    blocks, block_size, _, H, D = raw_pages.shape
    B = new_k.shape[0]
    if new_k.shape != (B, H, D) or new_v.shape != (B, H, D) or new_k.stride()[1:] != (D, 1) or \
            new_v.stride()[1:] != (D, 1):
        raise ValueError('new_k / new_v must be [B, Hkv, D] with contiguous heads')
    raw_table = _table(raw_table, raw_pages.device)
    beacon_table = _table(beacon_table, raw_pages.device) if sink else None
    if raw_table.shape[0] != B or (sink and beacon_table.shape[0] != B):
        raise ValueError('one table row per request')
    if cos.dtype != torch.float32 or sin.shape != cos.shape or cos.dim() != 2 or cos.shape[1] != D:
        raise ValueError('RoPE tables must be fp32 [rows, head_dim]')
    cos, sin = cos.contiguous(), sin.contiguous()
    positions = positions.to(torch.int64)
    positions = positions if positions.stride(-1) == 1 else positions.contiguous()
    if positions.shape[0] != B or positions.shape[1] < rows:
        raise ValueError('positions must be [B, >= rows]')
    window_start = window_start.to(device=raw_pages.device, dtype=torch.int64).contiguous()
    raw_count = raw_count.to(device=raw_pages.device, dtype=torch.int32).contiguous()
    per_request = [window_start, raw_count] + ([raw_write_end] if flush else []) + \
        ([sink_update] if flush and sink else [])
    if any(t is None or t.numel() < B for t in per_request):
        raise ValueError('window_start, raw_count (and with flush raw_write_end, sink_update) need an entry per request')
    if out_k is None:
        out_k = torch.empty(B, rows, H, D, dtype=BF16, device=raw_pages.device)
    if out_v is None:
        out_v = torch.empty_like(out_k)
    for t in (out_k, out_v):
        if t.shape != (B, rows, H, D) or t.stride()[2:] != (D, 1):
            raise ValueError('outputs must be [B, rows, Hkv, D] with contiguous heads')
    if flush:
        raw_write_end = raw_write_end.to(device=raw_pages.device, dtype=torch.int32).contiguous()
        if sink:
            sink_update = sink_update.to(device=raw_pages.device, dtype=torch.uint8).contiguous()
    status, owned = _status_word(status, raw_pages.device)
    st = raw_pages.stride()
    a = _lib.PagedStepRowsArgs(
        raw_pages=_ptr(raw_pages), num_blocks=blocks, p_sblk=st[0], p_stok=st[1], p_skind=st[2], p_sh=st[3],
        raw_table=_ptr(raw_table), rt_sb=raw_table.stride(0), rt_cols=raw_table.shape[1], block_size=block_size,
        beacon_pages=_ptr(beacon_pages) if sink else None,
        num_pages=beacon_pages.shape[0] if sink else 0,
        page_stride=(beacon_pages.stride(0) if page_stride is None else page_stride) if sink else 0,
        beacon_table=_ptr(beacon_table), bt_sb=beacon_table.stride(0) if sink else 0,
        new_k=_ptr(new_k), nk_sb=new_k.stride(0), new_v=_ptr(new_v), nv_sb=new_v.stride(0),
        window_start=_ptr(window_start), raw_count=_ptr(raw_count),
        positions=_ptr(positions), pos_sb=positions.stride(0),
        cos=_ptr(cos), sin=_ptr(sin), rope_rows=cos.shape[0],
        out_k=_ptr(out_k), ok_sb=out_k.stride(0), ok_sn=out_k.stride(1),
        out_v=_ptr(out_v), ov_sb=out_v.stride(0), ov_sn=out_v.stride(1),
        batch=B, rows=rows, kv_heads=H, head_dim=D, sink=int(sink), flush=int(bool(flush)),
        raw_write_end=_ptr(raw_write_end) if flush else None, sink_update=_ptr(sink_update) if flush and sink else None,
        status=_ptr(status))
    check(lib().slimkv_paged_step_rows(ctypes.byref(a), _lib.stream_handle(raw_pages.device)))
    if owned:
        check_status(status)
    return out_k, out_v


def raw_pages(pages, table, dense_k, dense_v, *, start, count, to_pages, lengths=None, status=None, starts=None):
    """Copy raw K/V between pages [blocks, block_size, 2, Hkv, D] and dense
    dense_k/dense_v [B, Hkv, count, D] (slimkv/vllm_plugin/paged_cache.py:102-127).
    Table entries, `status` and `starts` (request b's dense row r is position
    start + starts[b] + r) as beacon_pages."""
    _need_device(pages, dense_k, dense_v)
    _need_bf16(pages, dense_k, dense_v)
    if pages.dim() != 5 or pages.shape[2] != 2 or pages.stride(4) != 1:
        raise ValueError('pages must be [blocks, block_size, 2, heads, dim] with contiguous dim')
    table = _table(table, pages.device)
    B = table.shape[0]
    _, block_size, _, H, D = pages.shape
    for t in (dense_k, dense_v):
        if t.dim() != 4 or t.shape != (B, H, count, D) or t.stride(3) != 1:
            raise ValueError(f'dense K/V must be [{B}, {H}, {count}, {D}] with contiguous rows')
    lengths = _lengths(lengths, B, pages.device)
    starts = _starts(starts, B, pages.device)
    status, owned = _status_word(status, pages.device)
    a = _lib.RawPagesArgs(
        pages=_ptr(pages), num_blocks=pages.shape[0], p_sblk=pages.stride(0), p_stok=pages.stride(1),
        p_skind=pages.stride(2), p_sh=pages.stride(3),
        table=_ptr(table), t_sb=table.stride(0), t_cols=table.shape[1],
        dense_k=_ptr(dense_k), dk_sb=dense_k.stride(0), dk_sh=dense_k.stride(1), dk_sn=dense_k.stride(2),
        dense_v=_ptr(dense_v), dv_sb=dense_v.stride(0), dv_sh=dense_v.stride(1), dv_sn=dense_v.stride(2),
        lengths=_ptr(lengths), batch=B, start=start, count=count, block_size=block_size, kv_heads=H,
        head_dim=D, to_pages=int(bool(to_pages)), status=_ptr(status), starts=_ptr(starts))
    check(lib().slimkv_raw_pages(ctypes.byref(a), _lib.stream_handle(pages.device)))
    if owned:
        check_status(status)
