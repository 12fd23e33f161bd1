"""Drop-in for slimkv.llama3.paired_decode (the two-query insertion step).

original_splits restates slimkv/llama3/paired_decode.py:7-28 (host arithmetic,
kept for callers that size FA2 launches with it).

paired_attention (:30-43): the reference runs the insertion step's causal Q2
attention as two Q1 sequences over one K/V view (lengths [N-1, N]) with the
split count FA2 would pick for the unpacked Q2 launch, so that the packed
launch keeps the unpacked one's reduction order.  The HIP attention takes the
two queries of a step natively (GQA rows packed with both query positions), so
here the unpacked bottom-right causal Q2 launch itself is made: the raw query
sees N - 1 keys, the Beacon query N, and the result has, by construction, the
bits of the non-paired causal call (StaticDecode.attention's other branch,
static_decode.py:86-90).  No FA2 split heuristic is involved.
"""
import math
from functools import lru_cache


@lru_cache(None)
def original_splits(width, key_length, query_heads, sm_count):
    blocks = (key_length + 63) // 64
    if width == 320:
        splits = min(32, blocks, (sm_count + query_heads - 1) // query_heads)
        while splits > 1 and (splits - 1) * ((blocks + splits - 1) // splits) >= blocks:
            splits -= 1
        return splits
    sms = 2 * sm_count
    if query_heads >= 0.8 * sms:
        return 1
    block_n = 128 if width <= 128 else 64
    blocks = (key_length + block_n - 1) // block_n
    scores = {}
    for splits in range(1, min(128, sms, blocks) + 1):
        if splits > 1 and math.ceil(blocks / splits) == math.ceil(blocks / (splits - 1)):
            continue
        waves = query_heads * splits / sms
        scores[splits] = waves / math.ceil(waves)
    best = max(scores.values())
    return next(splits for splits, score in scores.items() if score >= 0.85 * best)


def paired_attention(forward, q, k, v, scale, paired_lengths, sm_count):
    """q [1, 2, H, W] (raw query, then the Beacon query), k/v [1, N_cap, Hk, W];
    paired_lengths: device int32 [N - 1, N] as StaticDecode fills it
    (static_decode.py:223-224) -- the Beacon query sees one key more.  Returns
    (out [1, 2, H, W], lse [1, H, 2]).  `sm_count` is not needed."""
    if q.shape[:2] != (1, 2) or k.shape[0] != 1:
        raise ValueError('Paired decode requires B1 and exactly two queries.')
    output, lse = forward(q, k, v, scale, True, 0, True, paired_lengths[1:])
    return output, lse
