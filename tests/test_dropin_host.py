"""Host-side behaviour of the drop-in modules (no GPU): gates, bookkeeping,
error behaviour, and the absence of any CPU compute fallback."""
from types import SimpleNamespace

import pytest
import torch

from oracle import splits as osplits


def test_backend_selection_matches_reference_table():
    # slimkv tests/test_llama_latent_eager.py:69-76
    from slimkv_amd.latent_decode import uses_fa2_decode, uses_latent_decode
    for backend, implementation, expected in [('latent', 'eager', False), ('latent', 'flash_attention_2', True),
                                              ('fa2', 'eager', True), ('reconstruct', 'eager', False)]:
        config = SimpleNamespace(beacon_decode_backend=backend, _attn_implementation=implementation)
        assert uses_fa2_decode(config) == expected
        assert uses_latent_decode(config) == (backend != 'reconstruct')


def test_original_splits_known_answers_and_oracle_agreement():
    from slimkv_amd.paired_decode import original_splits
    for length in [8256, 16448, 32832]:
        assert original_splits(320, length, 32, 78) == 3
        assert original_splits(256, length, 32, 78) == 9
    for width in (128, 200, 256, 320):
        for length in (64, 1000, 40000):
            for heads in (4, 32, 256):
                assert original_splits(width, length, heads, 78) == osplits.original_splits(width, length, heads, 78)


def test_paired_attention_rejects_other_shapes():
    from slimkv_amd.paired_decode import paired_attention
    with pytest.raises(ValueError):
        paired_attention(None, torch.zeros(2, 2, 4, 8), torch.zeros(1, 3, 1, 8), torch.zeros(1, 3, 1, 8), 1.0,
                         None, 78)


def test_fused_ops_defer_to_caller_off_gpu_and_kernels_refuse_cpu():
    from slimkv_amd import kernels
    from slimkv_amd.decode_ops import fused_merge, fused_rope
    from slimkv_amd.fa2_decode import merge_attention
    q = torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 3, 128, dtype=torch.bfloat16)
    assert fused_rope(q, k, None, None, None, 0, 0) is None                       # reference contract: torch path
    assert fused_merge(q, torch.zeros(1, 4, 1), q, torch.zeros(1, 4, 1)) is None
    with pytest.raises(ValueError):
        merge_attention(q, torch.zeros(1, 4, 1), q, torch.zeros(1, 4, 1))      # no CPU compute in the product
    with pytest.raises(ValueError):
        kernels.attention_forward(q.transpose(1, 2), k.transpose(1, 2), k.transpose(1, 2), 0.1)


def test_eager_forward_refuses_cpu_tensors():
    """The reference's eager_forward also runs on the CPU; this library has no
    CPU path, so CPU tensors raise before anything is launched."""
    from slimkv_amd.latent_decode import eager_forward
    q = torch.zeros(1, 1, 4, 32)
    k = torch.zeros(1, 3, 2, 32)
    with pytest.raises(ValueError, match='GPU'):
        eager_forward(q, k, k, 0.1)
    with pytest.raises(ValueError, match='shapes'):
        eager_forward(q, k[..., :16], k, 0.1)


def test_prepare_metadata_gate():
    from slimkv_amd.prefill_ops import prepare_metadata
    config = SimpleNamespace(beacon_prefill_fast=True, _slimkv_decode_step=False,
                             _attn_implementation='flash_attention_2', beacon_pos='interleave',
                             beacon_parallel_window=1, beacon_window=8, beacon_stride=8,
                             beacon_skip_rope_for_beacon_k=True)
    model = SimpleNamespace(config=config, training=False, memory=SimpleNamespace(latent_cache_active=True))
    roles = torch.tensor([0, 0, 1, 0, 2, 0])
    past = [(None, None, 1, roles)]
    with torch.no_grad():
        # CPU ids: the reference declines (prefill_ops.py:19-22) and so do we
        assert prepare_metadata(model, torch.zeros(1, 4, dtype=torch.long), None, None, past, None) is None


def test_block_diagonal_detection_is_exact():
    from slimkv_amd.memory import is_block_diagonal
    w = torch.zeros(4 * 8, 4 * 3)
    for h in range(4):
        w[h * 8:(h + 1) * 8, h * 3:(h + 1) * 3] = torch.randn(8, 3)
    assert is_block_diagonal(w, 4)
    w[0, 5] = 1e-30
    assert not is_block_diagonal(w, 4)                 # cached per version: the edit bumped it
    assert not is_block_diagonal(torch.randn(32, 12), 4)


def test_extension_module_signature():
    import inspect
    import sys
    sys.path.insert(0, 'slimkv_amd/fa2ext')
    import slimkv_fa2_decode_320 as ext
    assert ext.supports_cache_seqlens is True
    params = list(inspect.signature(ext.forward).parameters)
    assert params == ['q', 'k', 'v', 'softmax_scale', 'causal', 'num_splits', 'pack_q', 'cache_seqlens']
    with pytest.raises(RuntimeError):
        ext.forward(torch.zeros(1, 1, 4, 128), torch.zeros(1, 2, 1, 128), torch.zeros(1, 2, 1, 128), 0.1)


def test_prefill_history_follows_the_memory():
    """PrefillHistory bookkeeping on the host: an empty past restarts the
    stream, a past whose sink/history lengths differ from the store's (or that
    holds open window rows) is refused, the window's rows are reserved after
    the held rows and the capacity is enforced."""
    from slimkv_amd.memory import ReconstructionCache
    from slimkv_amd.prefill import PrefillHistory
    store = PrefillHistory(2, 2, 128, 40, 'cpu')
    empty = ReconstructionCache(None, None, None, None, None, 2, 128, 'k')
    assert store.follows(empty, empty)
    cur = torch.randn(2, 2, 16, 128).to(torch.bfloat16)
    base, kr, vr = store.reserve(2, 16)
    kr.copy_(cur)
    vr.copy_(-cur)
    k, v = store.sets(16)
    assert base == 0 and k.shape == (2, 2, 16, 128) and torch.equal(k, cur) and torch.equal(v, -cur)
    att = SimpleNamespace(num_key_value_heads=2)
    store.append(att, None, None, sink_size=4)            # no beacons: only the sink is kept
    assert (store.sink, store.history) == (4, 0)
    sink = torch.zeros(2, 2, 4, 128)
    hist = torch.zeros(2, 1, 8, 256)
    past = ReconstructionCache(sink, hist, None, None, None, 2, 128, 'k')
    assert not store.follows(past, past)                 # the store holds no history yet
    store.history = 8
    assert store.follows(past, past)
    base, kr, _ = store.reserve(2, 16)
    kr.copy_(cur)
    k, _ = store.sets(16)
    assert base == 12 and k.shape[2] == 4 + 8 + 16 and torch.equal(k[:, :, 12:], cur)
    with_window = ReconstructionCache(sink, hist, torch.zeros(2, 2, 3, 128), None, None, 2, 128, 'k')
    assert not store.follows(with_window, with_window)
    with pytest.raises(ValueError, match='capacity'):
        store.reserve(2, 29)
    with pytest.raises(ValueError, match='capacity'):
        store.reserve(3, 16)
    # 12 held rows + 29 new beacons pass the 40-row capacity: refused before any launch
    with pytest.raises(ValueError, match='capacity'):
        store.append(att, torch.zeros(2, 29, 64), torch.zeros(2, 29, 64), sink_size=4)
    assert store.history == 8
    assert store.follows(empty, empty) and (store.sink, store.history) == (0, 0)
