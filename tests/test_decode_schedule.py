"""Decode-step bookkeeping on the host: the schedule that drives the
append-only caches against the oracle's restatement of LlamaMemory._step
(slimkv/llama3/memory.py:101-162) and update_memory (:233-278), plus the
closed-form invariants the reference's own tests rely on (beacons per window =
window / ratio, a beacon after every `ratio` raw tokens, keys counted as
positions)."""
import pytest

from oracle import paged as opaged
from oracle import schedule as osched


@pytest.mark.parametrize('window,ratio,sink,processed', [(16, 4, 1, 0), (16, 4, 1, 21), (1024, 8, 1, 32768),
                                                         (24, 8, 0, 5), (8, 2, 1, 7)])
def test_schedule_matches_oracle(window, ratio, sink, processed):
    from slimkv_amd.decode_state import DecodeSchedule
    ours = DecodeSchedule.after_prefill(window, ratio, sink, processed)
    raw, history, beacons = opaged.restore_counts(processed, window, ratio)
    assert ours.window_raw == raw and ours.history == history
    assert ours.window_raw + ours.window_beacons == len(opaged.window_roles(raw, ratio))
    oracle = osched.DecodeSchedule(window, ratio, start=ours.start, processed=processed, roles=ours.roles,
                                   remainder=ours.remainder, full=ours.is_full)
    mem = osched.LatentMemory(sink=['s'] * sink, history=[f'h{i}' for i in range(history)],
                              raw=[f'r{i}' for i in range(raw)], window=[f'w{i}' for i in range(ours.window_beacons)],
                              sink_size=sink)
    for step in range(3 * window + 5):
        plan = ours.step()
        want = oracle.step(mem.keys())
        assert (plan.size, plan.full, plan.key_length) == (want.size, want.full, want.key_length), step
        assert plan.raw_slot == len(mem.sink) + len(mem.raw)
        assert plan.latent_slot == len(mem.history) + len(mem.window)
        assert plan.position == mem.keys()
        mem.update(f't{step}', [f'b{step}'] * plan.size, want.full)
        assert ours.history == len(mem.history)
        # invariants: a beacon closes every `ratio` raw tokens; a full window holds window/ratio beacons
        assert want.roles[-1 - plan.size] == 0 and (plan.size == 0 or want.roles[-1] == 1)
        if want.full:
            assert want.roles.count(1) == window // ratio and want.roles.count(0) == window


def test_first_window_sink_follows_newest_token_until_history_exists():
    """update_memory refreshes the sink while there is no history (memory.py:248-253)."""
    mem = osched.LatentMemory(sink=['s'], sink_size=1)
    sched = osched.DecodeSchedule(4, 2)
    for t in range(6):
        step = sched.step(mem.keys())
        mem.update(f't{t}', ['b'] * step.size, step.full)
        if t < 4:
            assert mem.sink == [f't{t}']
    assert mem.sink == ['t3'] and len(mem.history) == 2      # frozen once the first window closed


def test_cache_bytes_groups():
    mem = osched.LatentMemory(sink=['s'], history=['h'] * 3, raw=['r'] * 2, window=['w'], sink_size=1)
    assert mem.cache_bytes(4096, 1024) == {'sink': 4096, 'raw': 8192, 'beacon': 3072, 'window_beacon': 1024}
