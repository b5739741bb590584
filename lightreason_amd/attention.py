"""Full-attention decode on the GPU: the gated attention that runs before the
MoE block in 10 of the 40 decoder layers of the 35B model.

* ``AttentionDecode`` -- a ``Qwen3_5MoeAttention``'s weights ([HF] 627-720)
  bound to ``lrmoe_attn_decode``: ``step`` runs one cached forward of 1..16
  tokens (q/gate, k, v projections, per-head q/k RMSNorm, the rotary
  embedding, the cache append, causal attention over the cache, the sigmoid
  gate, o_proj) and returns the module's output.
* ``fused_attention(model)`` -- a context manager under which every
  full-attention layer's cached forward of 1..16 tokens (batch 1) is one
  ``lrmoe_attn_decode`` call; the layer's cache rows then live in a
  preallocated buffer that the Transformers cache layer views, so the
  kernel appends in place and cropping (speculative rollback) keeps working.
  The reference runs this module stock (Transformers SDPA); prefill, batches
  and longer blocks run stock here too.

There is no CPU path: the calls raise when liblrmoe.so is missing.
"""

from __future__ import annotations

from contextlib import contextmanager

import torch

from . import _native

HIDDEN = 2048
HEADS = 16
KV_HEADS = 2
HEAD_DIM = 256
ROTARY = 64
MAX_TOKENS = _native.ATTN_MAX_TOKENS


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require(t: torch.Tensor, name: str, dtypes, shape, device=None) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.dtype not in dtypes:
        raise ValueError(f"{name} must be {' or '.join(map(str, dtypes))}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if t.device.type != "cuda" or (device is not None and t.device != device):
        raise ValueError(f"{name} must be on {device or 'a GPU'}, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


_WORKSPACES: dict = {}


def _workspace(device: torch.device) -> torch.Tensor:
    """Scratch for lrmoe_attn_decode on the current stream of `device` (sized
    for 16 tokens; one per stream, as calls sharing it must not overlap)."""
    key = (device, _stream(device))
    ws = _WORKSPACES.get(key)
    if ws is None:
        nbytes = int(_native.library().lrmoe_attn_workspace_bytes(MAX_TOKENS))
        ws = _WORKSPACES[key] = torch.empty(nbytes, dtype=torch.uint8, device=device)
    return ws


class AttentionDecode:
    """The weights of one full-attention layer of the 35B model for
    ``lrmoe_attn_decode``: q_proj [8192, 2048] (per head 256 query rows,
    then 256 gate rows), k_proj and v_proj [512, 2048], o_proj [2048, 4096],
    q_norm and k_norm [256], all bf16 on one GPU."""

    def __init__(self, *, q_proj, k_proj, v_proj, o_proj, q_norm, k_norm, eps: float = 1e-6):
        dev = q_proj.device
        bf = (torch.bfloat16,)
        self.q_proj = _require(q_proj, "q_proj", bf, (HEADS * 2 * HEAD_DIM, HIDDEN), dev)
        self.k_proj = _require(k_proj, "k_proj", bf, (KV_HEADS * HEAD_DIM, HIDDEN), dev)
        self.v_proj = _require(v_proj, "v_proj", bf, (KV_HEADS * HEAD_DIM, HIDDEN), dev)
        self.o_proj = _require(o_proj, "o_proj", bf, (HIDDEN, HEADS * HEAD_DIM), dev)
        self.q_norm = _require(q_norm, "q_norm", bf, (HEAD_DIM,), dev)
        self.k_norm = _require(k_norm, "k_norm", bf, (HEAD_DIM,), dev)
        self.eps = float(eps)
        self.device = dev

    @classmethod
    def from_module(cls, attn) -> "AttentionDecode":
        """Bind a Transformers ``Qwen3_5MoeAttention`` (weights referenced,
        not copied)."""
        cfg = attn.config
        rotary = int(attn.head_dim * cfg.rope_parameters.get("partial_rotary_factor", 1.0))
        dims = (cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, attn.head_dim, rotary,
                attn.q_proj.bias is None and attn.o_proj.bias is None, attn.scaling)
        if dims != (HIDDEN, HEADS, KV_HEADS, HEAD_DIM, ROTARY, True, HEAD_DIM ** -0.5):
            raise ValueError(f"lrmoe_attn_decode serves the 35B attention shape only, got {dims}")
        return cls(q_proj=attn.q_proj.weight, k_proj=attn.k_proj.weight, v_proj=attn.v_proj.weight,
                   o_proj=attn.o_proj.weight, q_norm=attn.q_norm.weight, k_norm=attn.k_norm.weight,
                   eps=attn.q_norm.eps)

    def step(self, hidden: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, k_cache: torch.Tensor,
             v_cache: torch.Tensor, length, *, out: torch.Tensor | None = None) -> torch.Tensor:
        """One cached forward of T = hidden.shape[0] (1..16) tokens after
        `length` cached positions: hidden [T, 2048] bf16; cos, sin [T, 64]
        bf16 (the model's position embeddings of the new positions);
        k_cache, v_cache [2, capacity, 256] bf16 (normed, rotated keys and
        values), into which positions length .. length + T - 1 are written.
        Returns out [T, 2048] bf16.

        ``length`` is an int, or a one-element int32 tensor on the device
        that the kernels read when they run (``lrmoe_attn_decode_at``): a
        captured call then serves a cache that grows between replays.  The
        caller keeps its value in [0, capacity - T]; outside that range the
        output rows are NaN."""
        dev = self.device
        T = hidden.shape[0] if hidden.dim() == 2 else -1
        if not 1 <= T <= MAX_TOKENS:
            raise ValueError(f"hidden must be [T, {HIDDEN}] with 1 <= T <= {MAX_TOKENS}, got {tuple(hidden.shape)}")
        _require(hidden, "hidden", (torch.bfloat16,), (T, HIDDEN), dev)
        _require(cos, "cos", (torch.bfloat16,), (T, ROTARY), dev)
        _require(sin, "sin", (torch.bfloat16,), (T, ROTARY), dev)
        capacity = k_cache.shape[1] if k_cache.dim() == 3 else -1
        _require(k_cache, "k_cache", (torch.bfloat16,), (KV_HEADS, capacity, HEAD_DIM), dev)
        _require(v_cache, "v_cache", (torch.bfloat16,), (KV_HEADS, capacity, HEAD_DIM), dev)
        on_device = isinstance(length, torch.Tensor)
        if on_device:
            _require(length, "length", (torch.int32,), (1,), dev)
            if capacity < T:
                raise ValueError(f"{T} tokens exceed the cache capacity {capacity}")
        elif not 0 <= length <= capacity - T:
            raise ValueError(f"length {length} + {T} tokens exceeds the cache capacity {capacity}")
        if out is None:
            out = torch.empty((T, HIDDEN), dtype=torch.bfloat16, device=dev)
        _require(out, "out", (torch.bfloat16,), (T, HIDDEN), dev)
        ws = _workspace(dev)
        _native.call("lrmoe_attn_decode_at" if on_device else "lrmoe_attn_decode", hidden.data_ptr(), T,
                     self.q_proj.data_ptr(), self.k_proj.data_ptr(), self.v_proj.data_ptr(), self.o_proj.data_ptr(),
                     self.q_norm.data_ptr(), self.k_norm.data_ptr(), self.eps, cos.data_ptr(), sin.data_ptr(),
                     k_cache.data_ptr(), v_cache.data_ptr(), capacity,
                     length.data_ptr() if on_device else int(length), out.data_ptr(), ws.data_ptr(), ws.numel(),
                     _stream(dev))
        return out

    def layer_step(self, residual: torch.Tensor, input_norm: torch.Tensor, input_eps: float, cos: torch.Tensor,
                   sin: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, length, *, out: torch.Tensor,
                   sum_out: torch.Tensor, norm_out: torch.Tensor | None = None) -> torch.Tensor:
        """The decoder layer's full-attention half in one call
        (``lrmoe_attn_decode_step``): residual [T, 2048] bf16 is normed with
        input_norm [2048] (applied as 1 + w) in the projection launch,
        ``out`` receives the attention output and ``sum_out``
        bf16(residual + out); ``norm_out`` (optional) the normed rows.
        Caches and ``length`` (int or int32 [1] device tensor) as ``step``.
        Returns sum_out."""
        dev = self.device
        T = residual.shape[0] if residual.dim() == 2 else -1
        if not 1 <= T <= MAX_TOKENS:
            raise ValueError(f"residual must be [T, {HIDDEN}] with 1 <= T <= {MAX_TOKENS}, got {tuple(residual.shape)}")
        _require(residual, "residual", (torch.bfloat16,), (T, HIDDEN), dev)
        _require(input_norm, "input_norm", (torch.bfloat16,), (HIDDEN,), dev)
        _require(cos, "cos", (torch.bfloat16,), (T, ROTARY), dev)
        _require(sin, "sin", (torch.bfloat16,), (T, ROTARY), dev)
        capacity = k_cache.shape[1] if k_cache.dim() == 3 else -1
        _require(k_cache, "k_cache", (torch.bfloat16,), (KV_HEADS, capacity, HEAD_DIM), dev)
        _require(v_cache, "v_cache", (torch.bfloat16,), (KV_HEADS, capacity, HEAD_DIM), dev)
        on_device = isinstance(length, torch.Tensor)
        if on_device:
            _require(length, "length", (torch.int32,), (1,), dev)
            if capacity < T:
                raise ValueError(f"{T} tokens exceed the cache capacity {capacity}")
        elif not 0 <= length <= capacity - T:
            raise ValueError(f"length {length} + {T} tokens exceeds the cache capacity {capacity}")
        for name, t in (("out", out), ("sum_out", sum_out)) + ((("norm_out", norm_out),) if norm_out is not None else ()):
            _require(t, name, (torch.bfloat16,), (T, HIDDEN), dev)
        ws = _workspace(dev)
        _native.call("lrmoe_attn_decode_step", residual.data_ptr(), T, input_norm.data_ptr(), float(input_eps),
                     self.q_proj.data_ptr(), self.k_proj.data_ptr(), self.v_proj.data_ptr(), self.o_proj.data_ptr(),
                     self.q_norm.data_ptr(), self.k_norm.data_ptr(), self.eps, cos.data_ptr(), sin.data_ptr(),
                     k_cache.data_ptr(), v_cache.data_ptr(), capacity, 0 if on_device else int(length),
                     length.data_ptr() if on_device else None, out.data_ptr(), sum_out.data_ptr(),
                     None if norm_out is None else norm_out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev))
        return sum_out


class _LayerBuffer:
    """Capacity-backed key and value rows of one cache layer: the layer's
    keys/values are kept as views [1, 2, length, 256] of k/v [1, 2, capacity,
    256]."""

    def __init__(self):
        self.k = None
        self.v = None

    def views(self, layer) -> bool:
        keys = getattr(layer, "keys", None)
        return (self.k is not None and isinstance(keys, torch.Tensor) and keys.data_ptr() == self.k.data_ptr()
                and keys.stride() == self.k.stride() and layer.values.data_ptr() == self.v.data_ptr())

    def reserve(self, layer, length: int, tokens: int) -> None:
        need = length + tokens
        if self.views(layer) and self.k.shape[2] >= need:
            return
        capacity = max(2 * need, need + 512)
        keys, values = layer.keys, layer.values
        k = keys.new_empty((1, KV_HEADS, capacity, HEAD_DIM))
        v = values.new_empty((1, KV_HEADS, capacity, HEAD_DIM))
        k[:, :, :length].copy_(keys)
        v[:, :, :length].copy_(values)
        self.k, self.v = k, v
        layer.keys, layer.values = k[:, :, :length], v[:, :, :length]


@contextmanager
def fused_attention(model):
    """Run every full-attention layer's cached forward of 1..16 tokens (batch
    1, the standard causal mask over the block) through lrmoe_attn_decode
    for the duration of the block; the first such step of a layer moves its
    cached rows into a buffer with room to grow (doubling when full)."""
    restore = []
    buffers: dict = {}

    def native_forward(attn, original):
        bound = AttentionDecode.from_module(attn)
        index = attn.layer_idx

        def forward(hidden_states, position_embeddings, attention_mask=None, past_key_values=None, **kwargs):
            T = hidden_states.shape[1]
            layers = getattr(past_key_values, "layers", None)
            layer = layers[index] if layers is not None and index < len(layers) else None
            keys = getattr(layer, "keys", None)
            if (layer is None or hidden_states.shape[0] != 1 or not 1 <= T <= MAX_TOKENS
                    or not isinstance(keys, torch.Tensor) or keys.dim() != 4 or keys.shape[0] != 1
                    or keys.shape[2] == 0):
                return original(hidden_states, position_embeddings, attention_mask,
                                past_key_values=past_key_values, **kwargs)
            length = keys.shape[2]
            buf = buffers.setdefault(index, _LayerBuffer())
            buf.reserve(layer, length, T)
            cos, sin = position_embeddings
            out = bound.step(hidden_states[0].contiguous(), cos[0].contiguous(), sin[0].contiguous(), buf.k[0],
                             buf.v[0], length)
            layer.keys = buf.k[:, :, :length + T]
            layer.values = buf.v[:, :, :length + T]
            return out.unsqueeze(0), None
        return forward

    try:
        for layer in model.model.layers:
            attn = getattr(layer, "self_attn", None)
            if attn is None:
                continue
            restore.append((attn, attn.__dict__.get("forward")))
            attn.forward = native_forward(attn, attn.forward)
        yield
    finally:
        for attn, previous in restore:
            if previous is None:
                del attn.forward
            else:
                attn.forward = previous
