"""Whole-model decode steps captured as HIP graphs over append-only latent caches.

Drop-in for slimkv/llama3/static_decode.py:43-287 (StaticDecode): the same
constructor, eligibility rule, `initialize`/`forward`/`run`/`commit` and the
same exchange with the model's memory (`run` reads the slots from the
past-cache lengths, `commit` publishes valid views back).  Per layer the
decode attention is one call of the fused latent decode over a
LatentDecodeCache (raw rows rotated once when appended, latents appended in
place), bounded by device-side lengths, so one captured graph per step shape
serves every later step.  Batches of sequences in lockstep are allowed; the
reference's stream is batch 1.
"""
import math

import torch

from . import kernels
from .decode_state import LatentDecodeCache
from .latent_decode import uses_fa2_decode


def _length(x):
    return 0 if x is None else x.shape[2]


def _tables(rope, device):
    cos, sin = rope.cos_cached, rope.sin_cached
    if cos.device != device or cos.dtype != torch.float32:
        cos, sin = cos.to(device, torch.float32), sin.to(device, torch.float32)
    return cos.contiguous(), sin.contiguous()


def _bf16_linear(m, rows):
    """nn.Linear with contiguous bf16 weight (and bias) that the decode
    projection kernels take for `rows` rows (out features a multiple of 128)."""
    return (isinstance(m, torch.nn.Linear) and m.weight.dtype == torch.bfloat16 and m.weight.is_contiguous()
            and m.out_features % 128 == 0 and m.in_features % 8 == 0 and rows <= 4
            and (m.bias is None or (m.bias.dtype == torch.bfloat16 and m.bias.is_contiguous())))


def _fused_qkv(attn, rows):
    """(weight, bias) of the layer's q/k/v projections concatenated for the
    one-launch decode projection (kernels.decode_qkv), or None when the layer
    does not fit it.  The weights are copied once, when the stream is built."""
    mods = (attn.q_proj, attn.k_proj, attn.v_proj)
    if attn.head_dim != 128 or not all(_bf16_linear(m, rows) for m in mods):
        return None
    if len({m.in_features for m in mods}) != 1 or len({m.bias is None for m in mods}) != 1:
        return None
    if (attn.q_proj.out_features != attn.num_heads * 128 or
            attn.k_proj.out_features != attn.num_key_value_heads * 128 or
            attn.v_proj.out_features != attn.num_key_value_heads * 128):
        return None
    with torch.no_grad():
        weight = torch.cat([m.weight for m in mods]).contiguous()
        bias = None if attn.q_proj.bias is None else torch.cat([m.bias for m in mods]).contiguous()
    return weight, bias


class StaticDecode:
    """Lockstep decode stream; unsupported calls keep the ordinary model path."""

    def __init__(self, model, capacity, raw_capacity=None, batch=1):
        self.model = model
        self.capacity = capacity
        self.graphs = {}
        self.epoch = None
        self.batch = batch
        device = model.device
        self.raw_capacity = max(model.config.beacon_window + model.config.beacon_sink_size + 1, raw_capacity or 0)
        self.positions = torch.zeros(batch, 2, dtype=torch.long, device=device)
        self.caches = []
        # The new token's q/k/v projection, key RoPE and raw-cache appends run as
        # one launch over concatenated weights, and the output projection of
        # the token's row as a weight-streaming kernel (kernels.decode_qkv /
        # linear_rows), where the layer's projections allow it.
        self.qkv = []
        self.o_rows = []
        for layer in model.model.layers:
            attn = layer.self_attn
            self.caches.append(LatentDecodeCache(
                batch, attn.num_key_value_heads, attn.head_dim, attn.beacon_k_up_proj.in_features,
                attn.beacon_v_up_proj.in_features, self.raw_capacity, capacity, device, attn.q_proj.weight.dtype))
            self.qkv.append(_fused_qkv(attn, batch))
            self.o_rows.append(_bf16_linear(attn.o_proj, batch))

    @staticmethod
    def eligible(model, ids, past, kwargs):
        """static_decode.py:94-117 without the extension check: the attention
        runs in this package's HIP library."""
        return (ids.is_cuda and ids.shape[1] in (1, 2)
                and not torch.is_grad_enabled() and uses_fa2_decode(model.config)
                and getattr(model.config, 'beacon_decode_graph', False)
                and getattr(model.config, 'beacon_decode_graph_full', True)
                and model.dtype == torch.bfloat16
                and model.config.beacon_sink_size in (0, 1)
                and model.memory._fast_decode_active
                and not kwargs.get('output_attentions') and not kwargs.get('output_hidden_states')
                and kwargs.get('labels') is None and kwargs.get('inputs_embeds') is None
                and kwargs.get('return_dict', True) is not False
                and all(type(layer.self_attn.rotary_emb).__name__ in
                        ('RotaryEmbedding', 'LinearScalingRotaryEmbedding', 'Llama3RotaryEmbedding')
                        for layer in model.model.layers)
                and all(past[0][0].shape[2] + ids.shape[1] <= layer.self_attn.rotary_emb.max_seq_len_cached
                        for layer in model.model.layers)
                and all(isinstance(layer.self_attn.beacon_k_up_proj, torch.nn.Linear)
                        and isinstance(layer.self_attn.beacon_v_up_proj, torch.nn.Linear)
                        for layer in model.model.layers))

    def initialize(self, past):
        """Copy the memory's cache into the append-only buffers (static_decode.py:118-138)."""
        for cache, layer, (pk, pv, _, _) in zip(self.caches, self.model.model.layers, past):
            sink, raw, history = _length(pk.sink), _length(pk.raw), _length(pk.history)
            device = cache.raw_k.device
            positions = torch.cat([torch.arange(sink, device=device),
                                   pk.window_raw_indices.to(device) + sink + history if raw
                                   else torch.empty(0, dtype=torch.long, device=device)])
            cos, sin = _tables(layer.self_attn.rotary_emb, device)
            bshd = lambda x: None if x is None else x.transpose(1, 2)
            flat = lambda x: None if x is None else (x[:, 0] if x.shape[1] == 1 else
                                                     x.transpose(1, 2).reshape(x.shape[0], x.shape[2], -1))
            cache.load(bshd(pk.sink), bshd(pv.sink), bshd(pk.raw), bshd(pv.raw), flat(pk.history), flat(pv.history),
                       flat(pk.window), flat(pv.window), cos, sin,
                       positions[None].expand(cache.raw_k.shape[0], -1).contiguous())
        self.epoch = self.model.memory._static_decode_epoch

    def forward(self, ids, positions, return_normalized_hidden=False):
        """One decode step of the whole model (static_decode.py:140-208)."""
        model = self.model
        size = ids.shape[1] - 1
        length = 1 + size
        hidden = model.model.embed_tokens(ids[:, :1])
        if size:
            hidden = torch.cat([hidden, model.model.beacon_embed_tokens(ids[:, 1:] - model.config.vocab_size)], dim=1)
        B = hidden.shape[0]
        for cache, layer, fused, o_rows in zip(self.caches, model.model.layers, self.qkv, self.o_rows):
            residual = hidden
            normalized = layer.input_layernorm(hidden)
            attn = layer.self_attn
            cos, sin = _tables(attn.rotary_emb, hidden.device)
            kl = vl = None
            if size:
                kd = attn.beacon_kv_down_proj if attn._use_shared_kv_down_proj() else attn.beacon_k_down_proj
                vd = attn.beacon_kv_down_proj if attn._use_shared_kv_down_proj() else attn.beacon_v_down_proj
                kl, vl = kd(normalized[:, 1:]), vd(normalized[:, 1:])
            if fused is not None:
                # q of the token (unrotated: the decode rotates it), its key
                # rotated and appended with its value in the same launch
                q = kernels.decode_qkv(normalized[:, 0], fused[0], fused[1], attn.num_heads,
                                       attn.num_key_value_heads, cos, sin, positions[:, 0], cache.raw_k, cache.raw_v,
                                       cache.raw_index, plain_k=cache.plain_k,
                                       status=cache.status).view(B, 1, attn.num_heads, 128)
                if size:
                    qb = attn.beacon_q_proj if 'q' in attn.config.beacon_param else attn.q_proj
                    q = torch.cat([q, qb(normalized[:, 1:]).view(B, size, attn.num_heads, 128)], dim=1)
                if size:
                    cache.write_latents(kl, vl)
                rotation = dict(q_positions=positions, cos=cos, sin=sin)
            else:
                q = attn.q_proj(normalized)
                if size and 'q' in attn.config.beacon_param:
                    q = torch.cat([q[:, :1], attn.beacon_q_proj(normalized[:, 1:])], dim=1)
                q = q.view(B, length, attn.num_heads, attn.head_dim)
                raw_k = attn.k_proj(normalized[:, :1]).view(B, 1, attn.num_key_value_heads, attn.head_dim)
                raw_v = attn.v_proj(normalized[:, :1]).view(B, 1, attn.num_key_value_heads, attn.head_dim)
                q_rot, k_rot = kernels.rope_decode(q.transpose(1, 2), raw_k.transpose(1, 2), cos, sin, positions,
                                                   None, 0, 0)
                cache.write(k_rot.transpose(1, 2), raw_k, raw_v, kl, vl)
                q = q_rot.transpose(1, 2)
                rotation = dict(q_positions=None, cos=None, sin=None)
            uk, uv = attn.beacon_k_up_proj, attn.beacon_v_up_proj
            out, _ = cache.attend(q, uk.weight, uv.weight, 1.0 / math.sqrt(attn.head_dim), size=size,
                                  up_k_bias=uk.bias, up_v_bias=uv.bias, **rotation)
            merged = out.reshape(B, length, attn.hidden_size)
            if o_rows:
                output = kernels.linear_rows(merged[:, 0], attn.o_proj.weight, attn.o_proj.bias)[:, None]
                if size:
                    ob = attn.beacon_o_proj if 'o' in attn.config.beacon_param else attn.o_proj
                    output = torch.cat([output, ob(merged[:, 1:])], dim=1)
            else:
                output = attn.o_proj(merged)
                if size and 'o' in attn.config.beacon_param:
                    beacon_output = attn.beacon_o_proj(merged)
                    output = torch.cat([output[:, :1], beacon_output[:, 1:]], dim=1)
            hidden = layer._decode_tail(output, residual)
        hidden = model.model.norm(hidden)
        return hidden if return_normalized_hidden else model.lm_head(hidden).float()

    def _plan(self, past, size):
        """Slots of this step from the memory's past-cache lengths (static_decode.py:212-217)."""
        from .decode_state import StepPlan
        pk = past[0][0]
        sink, history = _length(pk.sink), _length(pk.history)
        raw = sink + _length(pk.raw)
        latent = history + _length(pk.window)
        return StepPlan(size, bool(self.model.memory._is_full_window), raw, latent, 0, 0)

    def run(self, ids, positions, past, return_normalized_hidden=False):
        """Replay (capturing on first use) the graph of this step shape
        (static_decode.py:210-265), then publish the cache views."""
        size = ids.shape[1] - 1
        if self.epoch != self.model.memory._static_decode_epoch:
            self.initialize(past)
        plan = self._plan(past, size)
        for cache in self.caches:
            cache.prepare(plan)
        positions = positions[:, -ids.shape[1]:]
        key = (size, return_normalized_hidden, ids.shape[0])
        if key not in self.graphs:
            buffers = (ids.clone(), positions.clone())
            current = torch.cuda.current_stream(ids.device)
            stream = torch.cuda.Stream(device=ids.device)
            stream.wait_stream(current)
            with torch.cuda.stream(stream):
                for _ in range(2):
                    self.forward(*buffers, return_normalized_hidden=return_normalized_hidden)
            current.wait_stream(stream)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                output = self.forward(*buffers, return_normalized_hidden=return_normalized_hidden)
            current.wait_stream(stream)
            self.graphs[key] = graph, buffers, output
        graph, buffers, output = self.graphs[key]
        buffers[0].copy_(ids)
        buffers[1].copy_(positions)
        graph.replay()
        self.commit(past, size, plan)
        return output.clone()

    def commit(self, past, size, plan=None):
        """Advance the caches and publish valid views to the memory
        (static_decode.py:267-287); views are BHSD as the memory keeps them."""
        plan = plan or self._plan(past, size)
        memory = self.model.memory
        for i, (cache, layer) in enumerate(zip(self.caches, self.model.model.layers)):
            cos, sin = _tables(layer.self_attn.rotary_emb, cache.raw_k.device)
            refresh = cache.history == 0 and cache.sink > 0 and not memory._decode_uncompressed
            sink = cache.sink
            cache.commit(plan, refresh, cos, sin)
            raw_end = plan.raw_slot + 1
            latent_end = plan.latent_slot + size
            bhsd = lambda x: x.transpose(1, 2)
            memory.sink_activations[i] = (bhsd(cache.plain_k[:, :sink]), bhsd(cache.raw_v[:, :sink]))
            if plan.full:
                memory.beacon_activations[i] = (cache.lat_k[:, :latent_end].unsqueeze(1),
                                                cache.lat_v[:, :latent_end].unsqueeze(1))
                memory.raw_activations[i] = (None, None)
                memory.window_beacon_activations[i] = (None, None)
            else:
                history = cache.history
                memory.beacon_activations[i] = tuple(x[:, :history].unsqueeze(1) if history else None
                                                     for x in (cache.lat_k, cache.lat_v))
                memory.raw_activations[i] = (bhsd(cache.plain_k[:, sink:raw_end]), bhsd(cache.raw_v[:, sink:raw_end]))
                memory.window_beacon_activations[i] = tuple(x[:, history:latent_end].unsqueeze(1)
                                                            if latent_end > history else None
                                                            for x in (cache.lat_k, cache.lat_v))
        memory._window_roles = None if memory._is_full_window else memory._fast_window_roles
        memory._window_raw_indices = None if memory._is_full_window else memory._fast_window_raw_indices

    def check_status(self):
        """Raise IndexError if a captured step's cache append met a slot outside
        the caches (synchronises the host; prepare() refuses such a step before
        it runs, so this is a second check)."""
        for cache in self.caches:
            kernels.check_status(cache.status)

    def cache_bytes(self):
        """Logical persistent K/V bytes over all layers (memory.py:280-287)."""
        total = {}
        for cache in self.caches:
            for k, v in cache.cache_bytes().items():
                total[k] = total.get(k, 0) + v
        return total
