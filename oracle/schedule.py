"""Decode-step bookkeeping of the latent cache (oracle; test infrastructure).

Restates, in plain Python over counts and role lists, what one decode step of
the reference does to the window schedule and to the cache contents:

  LlamaMemory._step, fast decode path     slimkv/llama3/memory.py:101-162
  LlamaMemory.update_memory (latent)      slimkv/llama3/memory.py:233-278
  LlamaMemory.cache_bytes                 slimkv/llama3/memory.py:280-287

with one compression ratio (Memory.set_compression_ratio returns
beacon_ratio[0] for a single ratio, slimkv/memory.py:212-250) and stride ==
window.  Tokens are tracked as labels, so the tests can check which token's
K/V sits in which slot.
"""


class Step:
    def __init__(self, size, roles, raw_indices, key_length, full):
        self.size = size                  # beacons inserted after the raw token (0 or 1)
        self.roles = roles                # window roles after the step (0 raw, 1 beacon)
        self.raw_indices = raw_indices    # role positions of the window's raw tokens
        self.key_length = key_length      # past keys + new raw token + new beacons
        self.full = full                  # the step completes the window


class DecodeSchedule:
    """Window state: window start, open-window roles, interleave remainder."""

    def __init__(self, window, ratio, start=0, processed=0, roles=(), remainder=0, full=True):
        self.window, self.ratio = window, ratio
        self.start, self.processed = start, processed
        self.roles, self.remainder, self.is_full = list(roles), remainder, full

    def step(self, past_keys):
        """One raw token (memory.py:104-162).  past_keys: keys before the step."""
        end = self.processed + 1
        full = end >= self.start + self.window
        if self.is_full:
            roles, raw = [], []
        else:
            roles = list(self.roles)
            raw = [i for i, r in enumerate(roles) if r == 0]
        size = (self.remainder + 1) // self.ratio
        self.remainder = (self.remainder + 1) % self.ratio
        raw.append(len(roles))
        roles += [0] + [1] * size
        self.roles = roles
        self.is_full = full
        if full:
            self.start += self.window
        self.processed = end
        return Step(size, roles, raw, past_keys + 1 + size, full)


class LatentMemory:
    """Cache contents as token labels: sink, history beacons, window raw tokens,
    window beacons (memory.py:233-278)."""

    def __init__(self, sink=(), history=(), raw=(), window=(), sink_size=1):
        self.sink, self.history = list(sink), list(history)
        self.raw, self.window = list(raw), list(window)
        self.sink_size = sink_size

    def keys(self):
        return len(self.sink) + len(self.history) + len(self.raw) + len(self.window)

    def update(self, raw_token, beacons, full):
        raw = self.raw + [raw_token]
        window = self.window + list(beacons)
        if not self.history and self.sink_size > 0:
            self.sink = [raw_token][:self.sink_size]        # first-window sink refresh (:248-253)
        if full:
            self.history += window
            self.raw, self.window = [], []
        else:
            self.raw, self.window = raw, window

    def cache_bytes(self, raw_row_bytes, latent_row_bytes):
        """Logical persistent bytes per group (memory.py:280-287)."""
        return {'sink': len(self.sink) * raw_row_bytes, 'raw': len(self.raw) * raw_row_bytes,
                'beacon': len(self.history) * latent_row_bytes, 'window_beacon': len(self.window) * latent_row_bytes}
