"""Split-count heuristics of the reference decode extension (oracle).

dense_splits     kernels/fa2_decode/binding.cpp:17-33
splits_320       kernels/fa2_decode/binding.cpp:98-105
original_splits  slimkv/llama3/paired_decode.py:7-28
"""
import math


def dense_splits(grid, sms, blocks):
    if grid >= 0.8 * sms:
        return 1
    limit = min(128, sms, blocks)
    eff = [0.0] * limit
    best = 0.0
    for s in range(1, limit + 1):
        if s > 1 and math.ceil(blocks / s) == math.ceil(blocks / (s - 1)):
            continue
        waves = grid * s / sms
        eff[s - 1] = waves / math.ceil(waves)
        best = max(best, eff[s - 1])
    for s in range(1, limit + 1):
        if eff[s - 1] >= 0.85 * best:
            return s
    return 1


def splits_320(grid_heads, sm_count, key_length):
    blocks = (key_length + 63) // 64
    splits = min(32, blocks, (sm_count + grid_heads - 1) // grid_heads)
    while splits > 1 and (splits - 1) * ((blocks + splits - 1) // splits) >= blocks:
        splits -= 1
    return splits


def original_splits(width, key_length, query_heads, sm_count):
    if width == 320:
        return splits_320(query_heads, sm_count, key_length)
    block_n = 128 if width <= 128 else 64
    return dense_splits(query_heads, 2 * sm_count, (key_length + block_n - 1) // block_n)
