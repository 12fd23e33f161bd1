"""The `slimkv_fa2_decode_320` module the reference imports by name.

Point SLIMKV_FA2_DECODE_EXTENSION_DIR at this directory and the reference's
flash_forward, StaticDecode, paired decode and benchmark runtime
(slimkv/llama3/fa2_decode.py:25-30, static_decode.py:20-29) load this module;
`forward` keeps the pybind signature of kernels/fa2_decode/binding.cpp:123-130
and runs the gfx950 split-K attention.
"""
import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

from slimkv_amd import kernels  # noqa: E402

supports_cache_seqlens = True


def forward(q, k, v, softmax_scale, causal=False, num_splits=0, pack_q=True, cache_seqlens=None):
    """BSHD bf16 q [B,Lq,H,W], k/v [B,N,Hk,W] -> [out [B,Lq,H,W], lse fp32 [B,H,Lq]].

    binding.cpp:35-121: Lq in {1, 2}; Hq % Hk == 0; N > 0; optional device int32
    cache_seqlens [B].  `num_splits` 0 chooses automatically; `pack_q` is
    accepted for signature compatibility (GQA packing is how the kernel always
    tiles).  Fully masked rows report LSE -inf (the reference kernel reports
    +inf and its Python wrapper converts).
    """
    for name, t in (('q', q), ('k', k), ('v', v)):
        if not t.is_cuda:
            raise RuntimeError(f'CUDA tensors required ({name})')
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise RuntimeError('BSHD tensors required')
    if q.shape[1] not in (1, 2):
        raise RuntimeError('Decode supports one/two queries')
    if k.shape[1] <= 0:
        raise RuntimeError('Handle empty branches before calling FA2')
    if q.shape[1] == 1:
        causal = False
    out, lse = kernels.attention_forward(q, k, v, softmax_scale, causal, splits=num_splits, seqlens=cache_seqlens)
    return [out, lse]
