"""ctypes binding of the C ABI in include/slimkv_hip.h.

The shared library is the only compute path.  Loading fails loudly when it is
missing: there is no CPU or PyTorch fallback behind any entry point.
"""
import ctypes
import os
from functools import lru_cache
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / 'libslimkv_hip.so'

c_i64 = ctypes.c_int64
c_i32 = ctypes.c_int32
c_ptr = ctypes.c_void_p
c_f64 = ctypes.c_double


def _struct(name, fields):
    return type(name, (ctypes.Structure,), {'_fields_': fields})


def _i64s(*names):
    return [(n, c_i64) for n in names]


AttentionArgs = _struct('slimkv_attention_args', [
    ('q', c_ptr), *_i64s('q_sb', 'q_sl', 'q_sh'),
    ('k', c_ptr), *_i64s('k_sb', 'k_sn', 'k_sh'),
    ('v', c_ptr), *_i64s('v_sb', 'v_sn', 'v_sh'),
    ('out', c_ptr), *_i64s('o_sb', 'o_sl', 'o_sh'),
    ('lse', c_ptr),
    ('seqlens', c_ptr),
    *_i64s('batch', 'queries', 'heads', 'kv_heads', 'keys', 'width_k', 'width_v'),
    ('scale', c_f64),
    ('causal', c_i32),
    ('splits', c_i32),
])

LatentDecodeArgs = _struct('slimkv_latent_decode_args', [
    ('q', c_ptr), *_i64s('q_sb', 'q_sl', 'q_sh'),
    ('q_positions', c_ptr), ('pos_sb', c_i64),
    ('cos', c_ptr), ('sin', c_ptr), ('rope_rows', c_i64),
    ('raw_k', c_ptr), *_i64s('rk_sb', 'rk_sn', 'rk_sh'),
    ('raw_v', c_ptr), *_i64s('rv_sb', 'rv_sn', 'rv_sh'),
    ('raw_lengths', c_ptr),
    ('raw_keys', c_i64),
    ('lat_k', c_ptr), *_i64s('lk_sb', 'lk_sn'),
    ('lat_v', c_ptr), *_i64s('lv_sb', 'lv_sn'),
    ('lat_lengths', c_ptr),
    ('lat_keys', c_i64),
    ('lat_causal', c_i32),
    ('block_diagonal', c_i32),
    ('up_k', c_ptr), ('up_k_bias', c_ptr),
    ('up_v', c_ptr), ('up_v_bias', c_ptr),
    *_i64s('batch', 'queries', 'heads', 'kv_heads', 'head_dim', 'rank_k', 'rank_v'),
    ('scale', c_f64),
    ('out', c_ptr), *_i64s('o_sb', 'o_sl', 'o_sh'),
    ('lse', c_ptr),
    ('raw_splits', c_i32), ('lat_splits', c_i32),
    ('up_k_t', c_ptr),
    ('lat_k2', c_ptr), *_i64s('lk2_sb', 'lk2_sn'),
    ('lat_v2', c_ptr), *_i64s('lv2_sb', 'lv2_sn'),
    ('lat_split', c_i64),
])

ReconstructArgs = _struct('slimkv_reconstruct_args', [
    ('latent', c_ptr), *_i64s('l_sb', 'l_sn'),
    ('weight', c_ptr), ('bias', c_ptr),
    ('out', c_ptr), *_i64s('o_sb', 'o_sn', 'o_sh'),
    ('dst_rows', c_ptr),
    ('cos', c_ptr), ('sin', c_ptr), ('rope_rows', c_i64),
    ('positions', c_ptr), ('pos_sb', c_i64),
    *_i64s('batch', 'rows', 'rank', 'kv_heads', 'head_dim'),
    ('block_diagonal', c_i32),
])

ReconDecodeArgs = _struct('slimkv_recon_decode_args', [
    ('base', LatentDecodeArgs),
    ('beacon_positions', c_ptr), ('bpos_sb', c_i64),
    ('rope_pairs', c_ptr), ('rope_repeats', c_i32), ('rope_fp32', c_i32),
])

LinearRowsArgs = _struct('slimkv_linear_rows_args', [
    ('x', c_ptr), ('x_sm', c_i64), ('weight', c_ptr), ('bias', c_ptr), ('out', c_ptr), ('o_sm', c_i64),
    *_i64s('m', 'n', 'k'),
])

DecodeQKVArgs = _struct('slimkv_decode_qkv_args', [
    ('x', c_ptr), ('x_sm', c_i64), ('weight', c_ptr), ('bias', c_ptr), ('q', c_ptr), ('q_sm', c_i64),
    ('raw_k', c_ptr), ('plain_k', c_ptr), ('raw_v', c_ptr), *_i64s('c_sm', 'c_sn'),
    ('slot_index', c_ptr), ('cos', c_ptr), ('sin', c_ptr), ('rope_rows', c_i64),
    ('positions', c_ptr), ('pos_sm', c_i64), *_i64s('m', 'k', 'heads', 'kv_heads', 'head_dim'),
    ('capacity', c_i64), ('status', c_ptr),
])

PagedLatentDecodeArgs = _struct('slimkv_paged_latent_decode_args', [
    ('base', LatentDecodeArgs),
    ('pages', c_ptr), *_i64s('num_pages', 'page_stride'),
    ('table', c_ptr), *_i64s('t_sb', 't_cols'),
    *_i64s('slots', 'sink_elements', 'rows_total'),
    ('status', c_ptr),
    ('raw_pages', c_ptr), *_i64s('raw_num_blocks', 'raw_block_size'),
    *_i64s('raw_block_stride', 'raw_token_stride', 'raw_kind_stride', 'raw_head_stride'),
    ('raw_table', c_ptr), *_i64s('raw_t_sb', 'raw_t_cols'),
])

RopeDecodeArgs = _struct('slimkv_rope_decode_args', [
    ('q', c_ptr), *_i64s('q_sb', 'q_sh', 'q_ss'),
    ('k', c_ptr), *_i64s('k_sb', 'k_sh', 'k_ss'),
    ('out_q', c_ptr), ('out_k', c_ptr),
    ('cos', c_ptr), ('sin', c_ptr), ('rope_rows', c_i64),
    ('q_positions', c_ptr), ('pos_sb', c_i64),
    ('raw_indices', c_ptr), ('raw_index_count', c_i64),
    *_i64s('batch', 'heads', 'kv_heads', 'queries', 'keys', 'dim', 'sink', 'history'),
])

PrefillRopeArgs = _struct('slimkv_prefill_rope_args', [
    ('q', c_ptr), *_i64s('q_sb', 'q_sh', 'q_ss'),
    ('k', c_ptr), *_i64s('k_sb', 'k_sh', 'k_ss'),
    ('out_q', c_ptr), *_i64s('oq_sb', 'oq_sh', 'oq_ss'),
    ('out_k', c_ptr), *_i64s('ok_sb', 'ok_sh', 'ok_ss'),
    ('cos', c_ptr), ('sin', c_ptr), ('rope_rows', c_i64),
    ('positions', c_ptr), ('pos_sb', c_i64),
    ('roles', c_ptr), ('role_len', c_i64),
    *_i64s('batch', 'heads', 'kv_heads', 'queries', 'keys', 'dim', 'sink'),
    ('v', c_ptr), *_i64s('v_sb', 'v_sh', 'v_ss'),
    ('out_v', c_ptr), *_i64s('ov_sb', 'ov_sh', 'ov_ss'),
])

MergeArgs = _struct('slimkv_merge_args', [
    ('raw', c_ptr), *_i64s('r_sb', 'r_sh', 'r_sl'),
    ('latent', c_ptr), *_i64s('l_sb', 'l_sh', 'l_sl'),
    ('raw_lse', c_ptr), *_i64s('rl_sb', 'rl_sh', 'rl_sl'),
    ('latent_lse', c_ptr), *_i64s('ll_sb', 'll_sh', 'll_sl'),
    ('out', c_ptr),
    *_i64s('batch', 'heads', 'length', 'dim'),
])

EagerAttentionArgs = _struct('slimkv_eager_attention_args', [
    ('q', c_ptr), *_i64s('q_sb', 'q_sl', 'q_sh'),
    ('k', c_ptr), *_i64s('k_sb', 'k_sn', 'k_sh'),
    ('v', c_ptr), *_i64s('v_sb', 'v_sn', 'v_sh'),
    ('out', c_ptr), *_i64s('o_sb', 'o_sl', 'o_sh'),
    ('lse', c_ptr),
    ('scores', c_ptr),
    *_i64s('batch', 'queries', 'heads', 'kv_heads', 'keys', 'rank', 'rank_v'),
    ('scale', c_f64),
    ('dtype', c_i32),
    ('causal', c_i32),
])

# Element types of the dtype-generic entry points (SLIMKV_DTYPE_*).
DTYPE_BF16, DTYPE_F16, DTYPE_F32 = 0, 1, 2

PrefillAttentionArgs = _struct('slimkv_prefill_attention_args', [
    ('q', c_ptr), *_i64s('q_sb', 'q_sl', 'q_sh'),
    ('k', c_ptr), *_i64s('k_sb', 'k_sn', 'k_sh'),
    ('v', c_ptr), *_i64s('v_sb', 'v_sn', 'v_sh'),
    ('out', c_ptr), *_i64s('o_sb', 'o_sl', 'o_sh'),
    ('lse', c_ptr),
    ('seqlens_k', c_ptr),
    *_i64s('batch', 'queries', 'heads', 'kv_heads', 'keys', 'head_dim'),
    ('scale', c_f64),
    ('causal', c_i32),
    ('rope_pairs', c_ptr), ('rope_rows', c_i64),
    ('rope_repeats', c_i32),
    ('q_positions', c_ptr), ('qpos_sb', c_i64),
])

DownProjectArgs = _struct('slimkv_down_project_args', [
    ('x', c_ptr), *_i64s('x_sb', 'x_sl'),
    ('rows', c_ptr), *_i64s('row_count', 'length'),
    ('weight', c_ptr),
    ('out', c_ptr), *_i64s('o_sb', 'o_sn'),
    *_i64s('batch', 'in_features', 'out_features', 'blocks'),
])

PageRows = _struct('slimkv_page_rows', [
    ('pages', c_ptr), *_i64s('num_pages', 'page_stride'),
    ('table', c_ptr), *_i64s('t_sb', 't_cols'),
    *_i64s('slots', 'sink_elements', 'slot_width', 'column'),
    ('start', c_i64),
    ('status', c_ptr),
])

BeaconPagesArgs = _struct('slimkv_beacon_pages_args', [
    ('pages', c_ptr), *_i64s('num_pages', 'page_stride'),
    ('table', c_ptr), *_i64s('t_sb', 't_cols'),
    ('dense_k', c_ptr), *_i64s('dk_sb', 'dk_sn'),
    ('dense_v', c_ptr), *_i64s('dv_sb', 'dv_sn'),
    ('lengths', c_ptr),
    *_i64s('batch', 'start', 'count', 'slots', 'key_rank', 'value_rank', 'sink_elements'),
    ('to_pages', c_i32),
    ('status', c_ptr), ('starts', c_ptr),
])

RawPagesArgs = _struct('slimkv_raw_pages_args', [
    ('pages', c_ptr), *_i64s('num_blocks', 'p_sblk', 'p_stok', 'p_skind', 'p_sh'),
    ('table', c_ptr), *_i64s('t_sb', 't_cols'),
    ('dense_k', c_ptr), *_i64s('dk_sb', 'dk_sh', 'dk_sn'),
    ('dense_v', c_ptr), *_i64s('dv_sb', 'dv_sh', 'dv_sn'),
    ('lengths', c_ptr),
    *_i64s('batch', 'start', 'count', 'block_size', 'kv_heads', 'head_dim'),
    ('to_pages', c_i32),
    ('status', c_ptr), ('starts', c_ptr),
])

PagedStepRowsArgs = _struct('slimkv_paged_step_rows_args', [
    ('raw_pages', c_ptr), *_i64s('num_blocks', 'p_sblk', 'p_stok', 'p_skind', 'p_sh'),
    ('raw_table', c_ptr), *_i64s('rt_sb', 'rt_cols', 'block_size'),
    ('beacon_pages', c_ptr), *_i64s('num_pages', 'page_stride'),
    ('beacon_table', c_ptr), ('bt_sb', c_i64),
    ('new_k', c_ptr), ('nk_sb', c_i64),
    ('new_v', c_ptr), ('nv_sb', c_i64),
    ('window_start', c_ptr), ('raw_count', c_ptr),
    ('positions', c_ptr), ('pos_sb', c_i64),
    ('cos', c_ptr), ('sin', c_ptr), ('rope_rows', c_i64),
    ('out_k', c_ptr), *_i64s('ok_sb', 'ok_sn'),
    ('out_v', c_ptr), *_i64s('ov_sb', 'ov_sn'),
    *_i64s('batch', 'rows', 'kv_heads', 'head_dim', 'sink'),
    ('flush', c_i32),
    ('raw_write_end', c_ptr), ('sink_update', c_ptr),
    ('status', c_ptr),
])

# name -> (restype, argtypes)
SIGNATURES = {
    'slimkv_last_error': (ctypes.c_char_p, []),
    'slimkv_abi_version': (ctypes.c_int, []),
    'slimkv_attention_workspace': (ctypes.c_size_t, [ctypes.POINTER(AttentionArgs)]),
    'slimkv_attention_forward': (ctypes.c_int, [ctypes.POINTER(AttentionArgs), c_ptr, ctypes.c_size_t, c_ptr]),
    'slimkv_latent_decode_workspace': (ctypes.c_size_t, [ctypes.POINTER(LatentDecodeArgs)]),
    'slimkv_latent_decode': (ctypes.c_int, [ctypes.POINTER(LatentDecodeArgs), c_ptr, ctypes.c_size_t, c_ptr]),
    'slimkv_latent_decode_stages': (ctypes.c_int, [ctypes.POINTER(LatentDecodeArgs), ctypes.c_int, c_ptr,
                                                   ctypes.c_size_t, c_ptr]),
    'slimkv_latent_decode_noalloc': (ctypes.c_int, [ctypes.POINTER(LatentDecodeArgs), c_ptr]),
    'slimkv_paged_latent_decode_workspace': (ctypes.c_size_t, [ctypes.POINTER(PagedLatentDecodeArgs)]),
    'slimkv_paged_latent_decode': (ctypes.c_int, [ctypes.POINTER(PagedLatentDecodeArgs), c_ptr, ctypes.c_size_t,
                                                  c_ptr]),
    'slimkv_paged_latent_decode_stages': (ctypes.c_int, [ctypes.POINTER(PagedLatentDecodeArgs), ctypes.c_int, c_ptr,
                                                         ctypes.c_size_t, c_ptr]),
    'slimkv_prepare_latent_bases': (ctypes.c_int, [c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr]),
    'slimkv_prepare_rope_pairs': (ctypes.c_int, [c_ptr, c_ptr, c_i64, c_i64, c_ptr, c_ptr]),
    'slimkv_reconstruct': (ctypes.c_int, [ctypes.POINTER(ReconstructArgs), c_ptr]),
    'slimkv_reconstruct_pair': (ctypes.c_int, [ctypes.POINTER(ReconstructArgs), ctypes.POINTER(ReconstructArgs), c_ptr]),
    'slimkv_recon_decode_workspace': (ctypes.c_size_t, [ctypes.POINTER(ReconDecodeArgs)]),
    'slimkv_recon_decode': (ctypes.c_int, [ctypes.POINTER(ReconDecodeArgs), c_ptr, ctypes.c_size_t, c_ptr]),
    'slimkv_recon_decode_stages': (ctypes.c_int, [ctypes.POINTER(ReconDecodeArgs), ctypes.c_int, c_ptr,
                                                  ctypes.c_size_t, c_ptr]),
    'slimkv_rope_decode': (ctypes.c_int, [ctypes.POINTER(RopeDecodeArgs), c_ptr]),
    'slimkv_linear_rows': (ctypes.c_int, [ctypes.POINTER(LinearRowsArgs), c_ptr]),
    'slimkv_decode_qkv': (ctypes.c_int, [ctypes.POINTER(DecodeQKVArgs), c_ptr]),
    'slimkv_prefill_rope': (ctypes.c_int, [ctypes.POINTER(PrefillRopeArgs), c_ptr]),
    'slimkv_merge': (ctypes.c_int, [ctypes.POINTER(MergeArgs), c_ptr]),
    'slimkv_merge_typed': (ctypes.c_int, [ctypes.POINTER(MergeArgs), ctypes.c_int, c_ptr]),
    'slimkv_eager_attention': (ctypes.c_int, [ctypes.POINTER(EagerAttentionArgs), c_ptr]),
    'slimkv_prefill_attention': (ctypes.c_int, [ctypes.POINTER(PrefillAttentionArgs), c_ptr]),
    'slimkv_down_project_workspace': (ctypes.c_size_t, [ctypes.POINTER(DownProjectArgs)]),
    'slimkv_down_project': (ctypes.c_int, [ctypes.POINTER(DownProjectArgs), c_ptr, ctypes.c_size_t, c_ptr]),
    'slimkv_down_project_pair_workspace': (ctypes.c_size_t, [ctypes.POINTER(DownProjectArgs),
                                                             ctypes.POINTER(DownProjectArgs)]),
    'slimkv_down_project_pair': (ctypes.c_int, [ctypes.POINTER(DownProjectArgs), ctypes.POINTER(DownProjectArgs),
                                                c_ptr, ctypes.c_size_t, c_ptr]),
    'slimkv_down_project_to_pages': (ctypes.c_int, [ctypes.POINTER(DownProjectArgs), ctypes.POINTER(PageRows), c_ptr,
                                                    ctypes.c_size_t, c_ptr]),
    'slimkv_beacon_pages': (ctypes.c_int, [ctypes.POINTER(BeaconPagesArgs), c_ptr]),
    'slimkv_raw_pages': (ctypes.c_int, [ctypes.POINTER(RawPagesArgs), c_ptr]),
    'slimkv_paged_step_rows': (ctypes.c_int, [ctypes.POINTER(PagedStepRowsArgs), c_ptr]),
}

ABI_VERSION = 15

STAGE_PROLOGUE, STAGE_ATTEND, STAGE_COMBINE, STAGE_ALL = 1, 2, 4, 7
NOALLOC_SCRATCH_BYTES = 32 << 20
STATUS_BAD_PAGE = 1
STATUS_BAD_SLOT = 2


class SlimKVError(RuntimeError):
    """A native entry point rejected its arguments or failed to launch."""


def library_path():
    """The library file lib() loads: the in-tree build, or the file the
    SLIMKV_HIP_LIBRARY environment variable names (an override for A/B runs)."""
    return Path(os.environ.get('SLIMKV_HIP_LIBRARY', LIBRARY))


def library_identity():
    """{'path', 'sha256', 'override'} of the library file lib() loads, for
    measurement records: which build a figure was taken on."""
    import hashlib
    path = library_path()
    digest = hashlib.sha256(path.read_bytes()).hexdigest() if path.exists() else None
    try:
        shown = str(path.resolve().relative_to(LIBRARY.parent.parent))
    except ValueError:
        shown = str(path)
    return {'path': shown, 'sha256': digest, 'override': 'SLIMKV_HIP_LIBRARY' in os.environ}


PROBE_LIBRARY = LIBRARY.with_name('libslimkv_probe.so')

PROBE_SIGNATURES = {
    'slimkv_probe_last_error': (ctypes.c_char_p, []),
    'slimkv_probe_stream_read': (ctypes.c_int, [c_ptr, c_i64, c_ptr, c_i64, c_i32, c_i32, c_i32, c_ptr]),
    'slimkv_probe_lds_read': (ctypes.c_int, [c_ptr, c_i64, c_i32, c_i32, c_i32, c_ptr]),
    'slimkv_probe_gather_read': (ctypes.c_int, [c_ptr, c_i64, c_ptr, c_i64, c_i64, c_i64, c_i32, c_ptr, c_i64,
                                                c_i32, c_ptr]),
    'slimkv_probe_touch': (ctypes.c_int, [c_ptr, c_i64, c_i32, c_ptr]),
}


@lru_cache(None)
def probe_lib():
    """The measurement probes (include/slimkv_probe.h), a library of their own
    beside the serving one."""
    if not PROBE_LIBRARY.exists():
        raise ImportError(f'{PROBE_LIBRARY} is missing: build it with `python -m slimkv_amd.build`')
    handle = ctypes.CDLL(str(PROBE_LIBRARY))
    for name, (restype, argtypes) in PROBE_SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle


def probe_check(code):
    if code != 0:
        raise SlimKVError(f'probe error {code}: {probe_lib().slimkv_probe_last_error().decode(errors="replace")}')


@lru_cache(None)
def lib():
    path = library_path()
    if not path.exists():
        raise ImportError(f'{path} is missing: build it with `python -m slimkv_amd.build` '
                          '(slimkv_amd has no fallback compute path)')
    handle = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if handle.slimkv_abi_version() != ABI_VERSION:
        raise ImportError(f'{path} has ABI {handle.slimkv_abi_version()}, expected {ABI_VERSION}')
    return handle


def check(code):
    if code != 0:
        message = lib().slimkv_last_error().decode(errors='replace')
        if code == -1:
            raise ValueError(message)
        raise SlimKVError(f'slimkv_hip error {code}: {message}')


def stream_handle(device):
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
