"""Drop-in for slimkv.llama3.latent_decode: backend selection and eager attention.

uses_latent_decode / uses_fa2_decode follow slimkv/llama3/latent_decode.py:7-13.
eager_forward keeps the reference signature (latent_decode.py:16-41) and runs
the HIP split-K attention, so a caller that selects the eager backend on the
GPU gets the same kernel as the FA2 backend; the fp32 CPU eager restatement
lives with the test oracle, not here.
"""


def uses_latent_decode(config):
    return getattr(config, 'beacon_decode_backend', 'reconstruct') in ('latent', 'fa2')


def uses_fa2_decode(config):
    backend = getattr(config, 'beacon_decode_backend', 'reconstruct')
    return backend == 'fa2' or (backend == 'latent' and config._attn_implementation == 'flash_attention_2')


def eager_forward(q, k, v, scale, causal=False):
    """BSHD inputs, BSHD output and BHQ log-sum-exp; K/V ranks may differ."""
    batch, queries, heads, rank = q.shape
    keys, kv_heads = k.shape[1:3]
    if (k.shape[0] != batch or k.shape[-1] != rank or v.shape[:3] != k.shape[:3]
            or kv_heads < 1 or heads % kv_heads or keys < 1):
        raise ValueError('Invalid eager attention shapes or GQA head counts.')
    from .fa2_decode import flash_forward
    out, lse = flash_forward(q, k, v, scale, causal)
    return out[..., :v.shape[-1]], lse
