"""Gated DeltaNet decode on the GPU: the linear-attention mixer that runs
before the MoE block in 30 of the 40 decoder layers of the 35B model.

* ``delta_rule(query, key, value, g, beta, initial, *, record, normalize)``
  -- the short-block gated delta rule with the calling convention of
  edge35b/delta_decode.py:38-55 (``_run``): one ``lrmoe_delta_rule`` launch.
* ``DeltaMixer`` -- a ``Qwen3_5MoeGatedDeltaNet``'s weights ([HF] 385-428)
  bound to ``lrmoe_delta_mixer``: ``step`` runs one cached forward of 1..16
  tokens ([HF] 430-543 with a previous state) as one persistent launch
  (in_proj with conv/beta/g, the delta rule, the gated RMSNorm, out_proj),
  updating the conv and recurrent states in place; ``mixer_status`` reads
  its timeout bit.
* ``PrefixStates`` -- the per-token states of the last recorded block of
  every linear-attention layer, and ``commit`` to roll the cache back to an
  accepted speculative prefix (delta_decode.py:58-81).
* ``fused_delta(model)`` -- a context manager (delta_decode.py:84-126) under
  which every linear-attention layer's cached forward of 1..16 tokens is one
  ``lrmoe_delta_mixer`` call on the live cache; other forwards (prefill, no
  cache, longer blocks, batches) run unchanged.  Blocks of 2..16 tokens
  inside ``histories.record(cache)`` keep per-token states for ``commit``.
  The reference patches only the recurrence into the stock forward and
  captures single-token forwards as graphs (packed_native.py:96-149);
  here the whole step is native and needs no capture or state copies.

There is no CPU path: the calls raise when liblrmoe.so is missing.
"""

from __future__ import annotations

from contextlib import contextmanager

import torch

from . import _native

HIDDEN = 2048
KEY_HEADS = 16
VALUE_HEADS = 32
HEAD_WIDTH = 128
CONV_DIM = 2 * KEY_HEADS * HEAD_WIDTH + VALUE_HEADS * HEAD_WIDTH  # 8192
CONV_TAPS = 4
MAX_TOKENS = _native.DELTA_MAX_TOKENS


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


def delta_rule(query, key, value, g, beta, initial, *, record: bool, normalize: bool):
    """The gated delta rule over a block (edge35b/delta_decode.py:38-55):
    query, key [1, T, H, D] bf16, value [1, T, H, E] bf16, g [1, T, H]
    (log decay; exp taken here as torch does), beta [1, T, H] bf16, initial
    [1, H, D, E] fp32 or bf16.  Returns (out [1, T, H, E] bf16, states
    [T if record else 1, H, D, E] in the state dtype)."""
    batch, steps, heads, key_width = query.shape
    value_width = value.shape[-1]
    if (batch != 1 or key_width not in (64, 128, 256) or value_width % 16
            or initial.shape != (batch, heads, key_width, value_width)
            or initial.dtype not in (torch.float32, torch.bfloat16)):
        raise ValueError(f"Unsupported recurrent layout {tuple(query.shape)}, {tuple(value.shape)}, "
                         f"{tuple(initial.shape)}, {initial.dtype}")
    device = query.device
    q = _require(query.contiguous(), "query", (torch.bfloat16,), (1, steps, heads, key_width), device)
    k = _require(key.contiguous(), "key", (torch.bfloat16,), (1, steps, heads, key_width), device)
    v = _require(value.contiguous(), "value", (torch.bfloat16,), (1, steps, heads, value_width), device)
    b = _require(beta.contiguous(), "beta", (torch.bfloat16,), (1, steps, heads), device)
    G = g.to(torch.float32).exp().contiguous()
    _require(G, "g", (torch.float32,), (1, steps, heads), device)
    init = _require(initial.contiguous(), "initial", (torch.float32, torch.bfloat16), initial.shape, device)
    out = torch.empty_like(v)
    states = init.new_empty((steps if record else 1, heads, key_width, value_width))
    _native.call("lrmoe_delta_rule", q.data_ptr(), k.data_ptr(), v.data_ptr(), G.data_ptr(), b.data_ptr(),
                 init.data_ptr(), int(init.dtype == torch.bfloat16), steps, heads, key_width, value_width,
                 int(bool(normalize)), int(bool(record)), out.data_ptr(), states.data_ptr(), _stream(device))
    return out, states


_WORKSPACES: dict = {}


def _workspace(device: torch.device) -> torch.Tensor:
    """Scratch for lrmoe_delta_mixer on the current stream of `device`
    (sized for 16 tokens, so its address never changes; one per stream, as
    calls sharing a workspace must not overlap; zeroed once, as its
    counters, flags and status word require)."""
    key = (device, _stream(device))
    ws = _WORKSPACES.get(key)
    if ws is None:
        nbytes = int(_native.library().lrmoe_delta_workspace_bytes(MAX_TOKENS))
        ws = _WORKSPACES[key] = torch.zeros(nbytes, dtype=torch.uint8, device=device)
    return ws


def check_mixer_status(device=None, what: str = "lrmoe_delta_mixer") -> int:
    """Raise RuntimeError when a mixer call on `device` (through any
    stream's workspace) had a bounded wait expire since the last check: the
    conv and recurrent states that call updated in place are invalid.  The
    timeout bit is sticky (every call ORs into the word), so it is cleared
    before raising and later calls report afresh.  Reads the device
    (synchronises); returns the OR of the status words otherwise."""
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    off = _native.DELTA_WS_STATUS_OFFSET
    status = 0
    for (dev, _stream_id), ws in list(_WORKSPACES.items()):
        if dev != device:
            continue
        word = ws[off:off + 4].view(torch.int32)
        value = int(word.item())
        if value & _native.STATUS_TIMEOUT:
            word.zero_()
        status |= value
    if status & _native.STATUS_TIMEOUT:
        raise RuntimeError(f"{what}: a cross-workgroup wait timed out, so the conv and recurrent states it updated "
                           "are invalid (the mixer kernel needs every workgroup resident: is another kernel "
                           "running on the device?)")
    return status


def mixer_status(device=None) -> int:
    """The status word of the current stream's mixer workspace (reads the
    device): LRMOE_STATUS_TIMEOUT once a call's bounded wait expired (its
    outputs invalid; a kernel on another stream kept workgroups off the
    GPU), 0 otherwise."""
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    ws = _workspace(device)
    off = _native.DELTA_WS_STATUS_OFFSET
    return int(ws[off:off + 4].view(torch.int32).item())


class DeltaMixer:
    """The weights of one Gated DeltaNet mixer of the 35B model for
    ``lrmoe_delta_mixer``: in_proj_qkv [8192, 2048], in_proj_z [4096, 2048],
    in_proj_b / in_proj_a [32, 2048], conv1d [8192, 4], A_log / dt_bias [32],
    norm [128], out_proj [2048, 4096], all bf16 on one GPU."""

    def __init__(self, *, in_proj_qkv, in_proj_z, in_proj_b, in_proj_a, conv1d, A_log, dt_bias, norm, out_proj,
                 eps: float = 1e-6):
        dev = in_proj_qkv.device
        bf = (torch.bfloat16,)
        self.in_proj_qkv = _require(in_proj_qkv, "in_proj_qkv", bf, (CONV_DIM, HIDDEN), dev)
        self.in_proj_z = _require(in_proj_z, "in_proj_z", bf, (VALUE_HEADS * HEAD_WIDTH, HIDDEN), dev)
        self.in_proj_b = _require(in_proj_b, "in_proj_b", bf, (VALUE_HEADS, HIDDEN), dev)
        self.in_proj_a = _require(in_proj_a, "in_proj_a", bf, (VALUE_HEADS, HIDDEN), dev)
        self.conv1d = _require(conv1d, "conv1d", bf, (CONV_DIM, CONV_TAPS), dev)
        self.A_log = _require(A_log, "A_log", bf, (VALUE_HEADS,), dev)
        self.dt_bias = _require(dt_bias, "dt_bias", bf, (VALUE_HEADS,), dev)
        self.norm = _require(norm, "norm", bf, (HEAD_WIDTH,), dev)
        self.out_proj = _require(out_proj, "out_proj", bf, (HIDDEN, VALUE_HEADS * HEAD_WIDTH), dev)
        self.eps = float(eps)
        self.device = dev

    @classmethod
    def from_module(cls, mixer) -> "DeltaMixer":
        """Bind a Transformers ``Qwen3_5MoeGatedDeltaNet`` (weights are
        referenced, not copied; conv1d.weight [8192, 1, 4] is viewed as
        [8192, 4])."""
        dims = (mixer.hidden_size, mixer.num_k_heads, mixer.num_v_heads, mixer.head_k_dim, mixer.head_v_dim,
                mixer.conv_kernel_size, mixer.activation, mixer.conv1d.bias is None)
        if dims != (HIDDEN, KEY_HEADS, VALUE_HEADS, HEAD_WIDTH, HEAD_WIDTH, CONV_TAPS, "silu", True):
            raise ValueError(f"lrmoe_delta_mixer serves the 35B mixer shape only, got {dims}")
        return cls(in_proj_qkv=mixer.in_proj_qkv.weight, in_proj_z=mixer.in_proj_z.weight,
                   in_proj_b=mixer.in_proj_b.weight, in_proj_a=mixer.in_proj_a.weight,
                   conv1d=mixer.conv1d.weight.squeeze(1), A_log=mixer.A_log, dt_bias=mixer.dt_bias,
                   norm=mixer.norm.weight, out_proj=mixer.out_proj.weight, eps=mixer.layer_norm_epsilon)

    def step(self, hidden: torch.Tensor, conv_state: torch.Tensor, state: torch.Tensor, *,
             conv_record: torch.Tensor | None = None, state_record: torch.Tensor | None = None,
             out: torch.Tensor | None = None) -> torch.Tensor:
        """One cached forward of T = hidden.shape[0] (1..16) tokens: hidden
        [T, 2048] bf16; conv_state [8192, 4] bf16 and state [32, 128, 128]
        (fp32 or bf16) are updated in place; conv_record [T, 8192, 4] and
        state_record [T, 32, 128, 128] (optional) receive both states after
        every token.  Returns out [T, 2048] bf16."""
        dev = self.device
        T = hidden.shape[0] if hidden.dim() == 2 else -1
        if not 1 <= T <= MAX_TOKENS:
            raise ValueError(f"hidden must be [T, {HIDDEN}] with 1 <= T <= {MAX_TOKENS}, got {tuple(hidden.shape)}")
        _require(hidden, "hidden", (torch.bfloat16,), (T, HIDDEN), dev)
        _require(conv_state, "conv_state", (torch.bfloat16,), (CONV_DIM, CONV_TAPS), dev)
        _require(state, "state", (torch.float32, torch.bfloat16), (VALUE_HEADS, HEAD_WIDTH, HEAD_WIDTH), dev)
        if conv_record is not None:
            _require(conv_record, "conv_record", (torch.bfloat16,), (T, CONV_DIM, CONV_TAPS), dev)
        if state_record is not None:
            _require(state_record, "state_record", (state.dtype,), (T, VALUE_HEADS, HEAD_WIDTH, HEAD_WIDTH), dev)
        if out is None:
            out = torch.empty((T, HIDDEN), dtype=torch.bfloat16, device=dev)
        _require(out, "out", (torch.bfloat16,), (T, HIDDEN), dev)
        ws = _workspace(dev)
        _native.call("lrmoe_delta_mixer", hidden.data_ptr(), T, self.in_proj_qkv.data_ptr(),
                     self.in_proj_z.data_ptr(), self.in_proj_b.data_ptr(), self.in_proj_a.data_ptr(),
                     self.conv1d.data_ptr(), self.A_log.data_ptr(), self.dt_bias.data_ptr(), self.norm.data_ptr(),
                     self.eps, self.out_proj.data_ptr(), conv_state.data_ptr(), state.data_ptr(),
                     int(state.dtype == torch.bfloat16),
                     None if conv_record is None else conv_record.data_ptr(),
                     None if state_record is None else state_record.data_ptr(),
                     out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev))
        return out

    def layer_step(self, residual: torch.Tensor, input_norm: torch.Tensor, input_eps: float,
                   conv_state: torch.Tensor, state: torch.Tensor, *, out: torch.Tensor,
                   sum_out: torch.Tensor, norm_out: torch.Tensor | None = None) -> torch.Tensor:
        """The decoder layer's linear-attention half in one launch
        (``lrmoe_delta_mixer_step``): residual [T, 2048] bf16 is normed with
        input_norm [2048] (the layer's input_layernorm, applied as 1 + w)
        inside the mixer, ``out`` receives the mixer output and ``sum_out``
        bf16(residual + out); ``norm_out`` (optional) the normed rows.
        States as ``step``.  Returns sum_out."""
        dev = self.device
        T = residual.shape[0] if residual.dim() == 2 else -1
        if not 1 <= T <= MAX_TOKENS:
            raise ValueError(f"residual must be [T, {HIDDEN}] with 1 <= T <= {MAX_TOKENS}, got {tuple(residual.shape)}")
        _require(residual, "residual", (torch.bfloat16,), (T, HIDDEN), dev)
        _require(input_norm, "input_norm", (torch.bfloat16,), (HIDDEN,), dev)
        _require(conv_state, "conv_state", (torch.bfloat16,), (CONV_DIM, CONV_TAPS), dev)
        _require(state, "state", (torch.float32, torch.bfloat16), (VALUE_HEADS, HEAD_WIDTH, HEAD_WIDTH), dev)
        for name, t in (("out", out), ("sum_out", sum_out)) + ((("norm_out", norm_out),) if norm_out is not None else ()):
            _require(t, name, (torch.bfloat16,), (T, HIDDEN), dev)
        ws = _workspace(dev)
        _native.call("lrmoe_delta_mixer_step", residual.data_ptr(), T, input_norm.data_ptr(), float(input_eps),
                     self.in_proj_qkv.data_ptr(), self.in_proj_z.data_ptr(), self.in_proj_b.data_ptr(),
                     self.in_proj_a.data_ptr(), self.conv1d.data_ptr(), self.A_log.data_ptr(), self.dt_bias.data_ptr(),
                     self.norm.data_ptr(), self.eps, self.out_proj.data_ptr(), conv_state.data_ptr(),
                     state.data_ptr(), int(state.dtype == torch.bfloat16), None, None, out.data_ptr(),
                     sum_out.data_ptr(), None if norm_out is None else norm_out.data_ptr(), ws.data_ptr(),
                     ws.numel(), _stream(dev))
        return sum_out


def _live(states):
    """The state tensor of a cache layer: Transformers 5.x keeps a dict
    {state_idx: tensor}, older versions the tensor itself."""
    return states[0] if isinstance(states, dict) else states


def _is_linear(layer) -> bool:
    return hasattr(layer, "conv_states") and hasattr(layer, "recurrent_states")


class PrefixStates:
    """Per linear-attention layer index, the conv and recurrent states after
    every token of the last block recorded inside ``record(cache)``
    (delta_decode.py:58-81 keeps the pre-block conv state and the block's
    projections instead; the conv state after token i is the same)."""

    def __init__(self):
        self.conv = {}
        self.recurrent = {}
        self.cache = None
        self.devices = set()  # devices whose mixer steps ran natively (status checked by commit)

    @contextmanager
    def record(self, cache):
        self.conv.clear()
        self.recurrent.clear()
        self.cache = cache
        try:
            yield
        finally:
            self.cache = None

    def commit(self, cache, prefix: int, accepted: int, width: int) -> None:
        """Keep the first `accepted` of the `width` positions verified after
        `prefix` cached tokens: attention layers are cut to prefix +
        accepted, linear-attention layers take the states recorded after
        position accepted - 1.  Nothing to do when all were accepted.
        First raises RuntimeError (check_mixer_status) when a native mixer
        step since the last check timed out: its states are invalid."""
        for device in self.devices:
            check_mixer_status(device, "fused_delta")
        if accepted == width:
            return
        if not 1 <= accepted < width or self.conv.keys() != self.recurrent.keys() or not self.conv:
            raise RuntimeError("Missing target state for the accepted speculative prefix")
        keep = prefix + accepted
        for layer in cache.layers:
            if _is_linear(layer) and not hasattr(layer, "keys"):
                continue
            length = layer.get_seq_length()
            if length > keep:
                layer.crop(keep - length)
        for index in self.conv:
            layer = cache.layers[index]
            _live(layer.conv_states)[0].copy_(self.conv[index][accepted - 1])
            _live(layer.recurrent_states)[0].copy_(self.recurrent[index][accepted - 1])


@contextmanager
def fused_delta(model):
    """Run every linear-attention layer's cached forward of 1..16 tokens
    (batch 1) through ``lrmoe_delta_mixer`` on the live cache for the
    duration of the block; yields the ``PrefixStates`` that blocks of
    2..16 tokens inside ``histories.record(cache)`` fill.  The mixer's
    status word is checked by every ``histories.commit`` and when the block
    ends without an exception: RuntimeError if a step timed out."""
    histories = PrefixStates()
    restore = []

    def native_forward(mixer, original, index):
        bound = DeltaMixer.from_module(mixer)

        def forward(hidden_states, cache_params=None, attention_mask=None, **kwargs):
            T = hidden_states.shape[1]
            if (cache_params is None or hidden_states.shape[0] != 1 or not 1 <= T <= MAX_TOKENS
                    or not cache_params.has_previous_state(index)
                    or getattr(cache_params.layers[index], "record_past", False)):
                return original(hidden_states, cache_params=cache_params, attention_mask=attention_mask, **kwargs)
            layer = cache_params.layers[index]
            conv = _live(layer.conv_states)[0]
            state = _live(layer.recurrent_states)[0]
            conv_rec = state_rec = None
            if histories.cache is not None and T > 1:
                conv_rec = torch.empty((T, CONV_DIM, CONV_TAPS), dtype=conv.dtype, device=conv.device)
                state_rec = torch.empty((T, *state.shape), dtype=state.dtype, device=state.device)
                histories.conv[index] = conv_rec
                histories.recurrent[index] = state_rec
            # batch 1: the padding mask leaves the states untouched ([HF] apply_mask_to_padding_states)
            out = bound.step(hidden_states[0].contiguous(), conv, state, conv_record=conv_rec, state_record=state_rec)
            histories.devices.add(conv.device)
            return out.unsqueeze(0)

        forward.lrmoe_native = True
        return forward

    try:
        for index, layer in enumerate(model.model.layers):
            mixer = getattr(layer, "linear_attn", None)
            if mixer is None:
                continue
            restore.append((mixer, mixer.__dict__.get("forward")))
            mixer.forward = native_forward(mixer, mixer.forward, index)
        yield histories
        for device in histories.devices:
            check_mixer_status(device, "fused_delta")
    finally:
        for mixer, previous in restore:
            if previous is None:
                del mixer.forward
            else:
                mixer.forward = previous
