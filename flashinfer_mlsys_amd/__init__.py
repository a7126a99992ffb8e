"""MI355X-native FP8 block-scale DeepSeek-V3 MoE operator (32 local experts).

Operator ``moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048``
(``reference moe/ref_moe.json``). The Python entry points keep the reference's
names and positional order:

* ``kernel(routing_logits, routing_bias, hidden_states, hidden_states_scale,
  gemm1_weights, gemm1_weights_scale, gemm2_weights, gemm2_weights_scale,
  local_expert_offset, routed_scaling_factor, output)`` -- destination-passing
  form of ``solution/triton/kernel.py:292-305``; writes ``output`` in place.
* ``run(...)`` -- the same ten inputs, returns the bf16 [T, 7168] output, as
  ``reference moe/ref_moe.py:4-16``.

Both validate the inputs the way ``ref_moe.py:41-63`` does (an
``AssertionError`` subclass on a geometry or dtype mismatch) and then call the
hand-written gfx950 HIP kernels in ``libmoe_mi355x.so`` through its C ABI on
the current HIP stream. There is no CPU or PyTorch fallback: a missing library
or a CPU tensor raises.

``route`` and ``dispatch`` expose the first two stages for parity tests.
"""
from __future__ import annotations

import torch

from . import _lib

__all__ = ["kernel", "run", "route", "dispatch", "route_dispatch", "quantize_activations", "router_logits",
           "router_logits_and_quantize", "workspace_size", "MoEInputError", "run_shape", "SHAPE_AUTO",
           "SHAPE_PREFILL"]

# Expert-GEMM kernel shapes for run_shape / route_dispatch (include/moe_fp8.h MOE_SHAPE_*):
# the decode kernels up to MOE_FP8_DECODE_MAX_TOKENS (96) tokens and the prefill kernels above, or the
# prefill kernels always.
SHAPE_AUTO = 0
SHAPE_PREFILL = 1

H = 7168
I = 2048
E_GLOBAL = 256
E_LOCAL = 32
BLOCK = 128
TOP_K = 8


class MoEInputError(AssertionError):
    """An input does not match the operator definition (shape, dtype, device)."""


def _req(cond, msg):
    if not cond:
        raise MoEInputError(msg)


def _on_gpu(t, name):
    # (the messages are formatted only on failure: this runs on every call)
    if not isinstance(t, torch.Tensor):
        raise MoEInputError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise MoEInputError(f"{name} must be on a ROCm GPU (got {t.device}); there is no CPU path")
    return t


# The current stream's raw handle for a device index (the accessor torch's own
# generated code uses; about a tenth of the cost of current_stream(...).cuda_stream).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device):
    if _raw_stream is not None:
        return _raw_stream(device.index if isinstance(device, torch.device) else int(device))
    return torch.cuda.current_stream(device).cuda_stream


def _contig(t):
    return t if t.is_contiguous() and t.data_ptr() % 16 == 0 else t.contiguous()


def _header_words(T: int) -> int:
    """MOE_FP8_DISPATCH_HEADER_WORDS(T): the header, then 32 counts per group of 16 tokens."""
    return _lib.MOE_FP8_HEADER_WORDS + 32 * ((T + 15) // 16)


def workspace_size(T: int) -> int:
    """Device workspace bytes ``kernel`` needs for T tokens."""
    return int(_lib.load().moe_fp8_workspace_size(int(T)))


def _validate(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
              gemm1_weights_scale, gemm2_weights, gemm2_weights_scale):
    names = ["routing_logits", "routing_bias", "hidden_states", "hidden_states_scale", "gemm1_weights",
             "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale"]
    ts = [routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
          gemm1_weights_scale, gemm2_weights, gemm2_weights_scale]
    for t, n in zip(ts, names):
        _on_gpu(t, n)
    dev = hidden_states.get_device()
    for t, n in zip(ts, names):
        if t.get_device() != dev:
            raise MoEInputError(f"{n} is on {t.device}, expected {hidden_states.device}")
    _req(routing_logits.dim() == 2, "routing_logits must be [T, 256]")
    T = routing_logits.shape[0]
    _req(routing_logits.shape[1] == E_GLOBAL, "num_experts must be 256")
    _req(gemm1_weights.dim() == 3 and gemm1_weights.shape[0] == E_LOCAL, "num_local_experts must be 32")
    _req(hidden_states.shape == (T, H), "hidden_size must be 7168")
    _req(hidden_states_scale.shape == (H // BLOCK, T), "hidden_states_scale must be [56, T]")
    _req(gemm1_weights.shape == (E_LOCAL, 2 * I, H), "intermediate_size must be 2048")
    _req(gemm1_weights_scale.shape == (E_LOCAL, 2 * I // BLOCK, H // BLOCK), "gemm1_weights_scale must be [32, 32, 56]")
    _req(gemm2_weights.shape == (E_LOCAL, H, I), "gemm2_weights must be [32, 7168, 2048]")
    _req(gemm2_weights_scale.shape == (E_LOCAL, H // BLOCK, I // BLOCK), "gemm2_weights_scale must be [32, 56, 16]")
    _req(routing_bias.shape[-1] == E_GLOBAL and routing_bias.numel() == E_GLOBAL, "routing_bias must have 256 entries")
    _req(routing_logits.dtype == torch.float32, "routing_logits must be float32")
    _req(routing_bias.dtype == torch.bfloat16, "routing_bias must be bfloat16")
    _req(hidden_states.dtype == torch.float8_e4m3fn, "hidden_states must be float8_e4m3fn")
    _req(gemm1_weights.dtype == torch.float8_e4m3fn, "gemm1_weights must be float8_e4m3fn")
    _req(gemm2_weights.dtype == torch.float8_e4m3fn, "gemm2_weights must be float8_e4m3fn")
    for t, n in ((hidden_states_scale, "hidden_states_scale"), (gemm1_weights_scale, "gemm1_weights_scale"),
                 (gemm2_weights_scale, "gemm2_weights_scale")):
        if t.dtype != torch.float32:
            raise MoEInputError(f"{n} must be float32")
    return T


def _forward(shape, routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
             gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
             routed_scaling_factor, output, workspace):
    T = _validate(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                  gemm1_weights_scale, gemm2_weights, gemm2_weights_scale)
    _on_gpu(output, "output")
    _req(output.shape == (T, H) and output.dtype == torch.bfloat16, "output must be bf16 [T, 7168]")
    _req(output.get_device() == hidden_states.get_device(), "output must be on the inputs' device")
    if T == 0:
        return None
    lib = _lib.load()
    need = int(lib.moe_fp8_workspace_size(T))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=hidden_states.device)
    _req(workspace.is_cuda and workspace.numel() * workspace.element_size() >= need, "workspace too small")
    args = [_contig(t) for t in (routing_logits, routing_bias.reshape(-1), hidden_states, hidden_states_scale,
                                 gemm1_weights, gemm1_weights_scale, gemm2_weights, gemm2_weights_scale)]
    out = output if (output.is_contiguous() and output.data_ptr() % 16 == 0) else torch.empty_like(
        output, memory_format=torch.contiguous_format)
    def call():
        tail = (T, int(local_expert_offset), float(routed_scaling_factor), out.data_ptr(), workspace.data_ptr(),
                workspace.numel() * workspace.element_size(), _stream(hidden_states.device))
        if shape == SHAPE_AUTO:
            return lib.moe_fp8_forward(*[a.data_ptr() for a in args], *tail)
        return lib.moe_fp8_forward_shape(int(shape), *[a.data_ptr() for a in args], *tail)

    if torch.cuda.current_device() == hidden_states.get_device():
        code = call()
    else:  # the library launches on the current device
        with torch.cuda.device(hidden_states.device):
            code = call()
    _lib.check(code, "moe_fp8_forward")
    if out is not output:
        output.copy_(out)
    return None


@torch.no_grad()
def kernel(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
           gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
           routed_scaling_factor, output, workspace=None):
    """Destination-passing operator: writes bf16 [T, 7168] into ``output``; returns None."""
    _forward(SHAPE_AUTO, routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
             gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset, routed_scaling_factor,
             output, workspace)


@torch.no_grad()
def run(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights, gemm1_weights_scale,
        gemm2_weights, gemm2_weights_scale, local_expert_offset, routed_scaling_factor):
    """Value-returning operator (``reference moe/ref_moe.py:4-16``): returns bf16 [T, 7168]."""
    _on_gpu(hidden_states, "hidden_states")
    T = routing_logits.shape[0]
    output = torch.empty((T, H), dtype=torch.bfloat16, device=hidden_states.device)
    kernel(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights, gemm1_weights_scale,
           gemm2_weights, gemm2_weights_scale, local_expert_offset, routed_scaling_factor, output)
    return output


@torch.no_grad()
def run_shape(shape, routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
              gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset, routed_scaling_factor):
    """``run`` with the expert-GEMM kernel shape chosen for this call (SHAPE_AUTO or
    SHAPE_PREFILL): tests run both shapes on the same inputs."""
    _req(shape in (SHAPE_AUTO, SHAPE_PREFILL), "shape must be SHAPE_AUTO or SHAPE_PREFILL")
    _on_gpu(hidden_states, "hidden_states")
    T = routing_logits.shape[0]
    output = torch.empty((T, H), dtype=torch.bfloat16, device=hidden_states.device)
    _forward(shape, routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
             gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset, routed_scaling_factor,
             output, None)
    return output


@torch.no_grad()
def route(routing_logits, routing_bias, routed_scaling_factor):
    """Routing stage: (topk_ids int32 [T, 8] ascending per token, topk_w fp32 [T, 8], tok_pair int32 [T, 8] = -1)."""
    _on_gpu(routing_logits, "routing_logits")
    _on_gpu(routing_bias, "routing_bias")
    _req(routing_logits.dtype == torch.float32 and routing_logits.dim() == 2
         and routing_logits.shape[1] == E_GLOBAL, "routing_logits must be float32 [T, 256]")
    _req(routing_bias.dtype == torch.bfloat16 and routing_bias.numel() == E_GLOBAL, "routing_bias must be bf16 [256]")
    T = routing_logits.shape[0]
    dev = routing_logits.device
    ids = torch.empty((T, TOP_K), dtype=torch.int32, device=dev)
    w = torch.empty((T, TOP_K), dtype=torch.float32, device=dev)
    pair = torch.empty((T, TOP_K), dtype=torch.int32, device=dev)
    if T == 0:
        return ids, w, pair
    lg, b = _contig(routing_logits), _contig(routing_bias.reshape(-1))
    with torch.cuda.device(dev):
        code = _lib.load().moe_fp8_route(lg.data_ptr(), b.data_ptr(), T, float(routed_scaling_factor),
                                         ids.data_ptr(), w.data_ptr(), pair.data_ptr(), _stream(dev))
    _lib.check(code, "moe_fp8_route")
    return ids, w, pair


@torch.no_grad()
def quantize_activations(hidden_bf16, out=None):
    """Producer-side FP8 quantiser: bf16 [T, 7168] -> (hidden_states e4m3 [T, 7168],
    hidden_states_scale fp32 [56, T]), the operator's own input format.

    Per 1 x 128 block: scale = max(amax, 1e-12) / 448, q = e4m3(x / scale) with
    round to nearest even (the reference's quantisation step,
    solution/triton/dsl-temp1.py:479-484). ``out`` may pass preallocated
    (q, scale) tensors.
    """
    _on_gpu(hidden_bf16, "hidden_bf16")
    _req(hidden_bf16.dtype == torch.bfloat16 and hidden_bf16.dim() == 2 and hidden_bf16.shape[1] == H,
         "hidden_bf16 must be bf16 [T, 7168]")
    T = hidden_bf16.shape[0]
    dev = hidden_bf16.device
    if out is None:
        q = torch.empty((T, H), dtype=torch.float8_e4m3fn, device=dev)
        scale = torch.empty((H // BLOCK, T), dtype=torch.float32, device=dev)
    else:
        q, scale = out
        _req(q.dtype == torch.float8_e4m3fn and tuple(q.shape) == (T, H) and q.is_contiguous(),
             "q must be a contiguous float8_e4m3fn [T, 7168]")
        _req(scale.dtype == torch.float32 and tuple(scale.shape) == (H // BLOCK, T) and scale.is_contiguous(),
             "scale must be a contiguous float32 [56, T]")
    if T == 0:
        return q, scale
    x = _contig(hidden_bf16)
    with torch.cuda.device(dev):
        code = _lib.load().moe_fp8_quantize_activations(x.data_ptr(), T, q.data_ptr(), scale.data_ptr(), _stream(dev))
    _lib.check(code, "moe_fp8_quantize_activations")
    return q, scale


@torch.no_grad()
def router_logits(hidden_bf16, gate_weight, out=None):
    """Router GEMM: routing_logits fp32 [T, 256] = hidden_bf16 [T, 7168] x gate_weight^T,
    gate_weight bf16 [256, 7168] (the linear layer that produces this operator's
    routing_logits, reference moe/weight_origins_dataflow.md:21, :151-154). Products
    are exact in fp32 and summed in fp32 in a fixed order. ``out`` may pass a
    preallocated fp32 [T, 256] tensor."""
    _on_gpu(hidden_bf16, "hidden_bf16")
    _on_gpu(gate_weight, "gate_weight")
    _req(hidden_bf16.dtype == torch.bfloat16 and hidden_bf16.dim() == 2 and hidden_bf16.shape[1] == H,
         "hidden_bf16 must be bf16 [T, 7168]")
    _req(gate_weight.dtype == torch.bfloat16 and tuple(gate_weight.shape) == (E_GLOBAL, H),
         "gate_weight must be bf16 [256, 7168]")
    _req(gate_weight.device == hidden_bf16.device, "gate_weight must be on the hidden states' device")
    T = hidden_bf16.shape[0]
    dev = hidden_bf16.device
    if out is None:
        out = torch.empty((T, E_GLOBAL), dtype=torch.float32, device=dev)
    else:
        _req(out.dtype == torch.float32 and tuple(out.shape) == (T, E_GLOBAL) and out.is_contiguous(),
             "out must be a contiguous float32 [T, 256]")
    if T == 0:
        return out
    x, g = _contig(hidden_bf16), _contig(gate_weight)
    lib = _lib.load()
    with torch.cuda.device(dev):
        code = lib.moe_fp8_router_logits(x.data_ptr(), g.data_ptr(), T, out.data_ptr(), _stream(dev))
    _lib.check(code, "moe_fp8_router_logits")
    return out


@torch.no_grad()
def router_logits_and_quantize(hidden_bf16, gate_weight, out=None):
    """The producer side (one pass over the bf16 hidden states below 576 tokens,
    the router and quantiser kernels in turn from 576 on): returns
    (routing_logits fp32 [T, 256], hidden_states e4m3 [T, 7168], hidden_states_scale
    fp32 [56, T]), bit for bit what ``router_logits`` and ``quantize_activations``
    return (reference moe/weight_origins_dataflow.md:19-21, :151-154). ``out`` may
    pass the three tensors preallocated."""
    _on_gpu(hidden_bf16, "hidden_bf16")
    _on_gpu(gate_weight, "gate_weight")
    _req(hidden_bf16.dtype == torch.bfloat16 and hidden_bf16.dim() == 2 and hidden_bf16.shape[1] == H,
         "hidden_bf16 must be bf16 [T, 7168]")
    _req(gate_weight.dtype == torch.bfloat16 and tuple(gate_weight.shape) == (E_GLOBAL, H),
         "gate_weight must be bf16 [256, 7168]")
    _req(gate_weight.device == hidden_bf16.device, "gate_weight must be on the hidden states' device")
    T = hidden_bf16.shape[0]
    dev = hidden_bf16.device
    if out is None:
        logits = torch.empty((T, E_GLOBAL), dtype=torch.float32, device=dev)
        q = torch.empty((T, H), dtype=torch.float8_e4m3fn, device=dev)
        scale = torch.empty((H // BLOCK, T), dtype=torch.float32, device=dev)
    else:
        logits, q, scale = out
        _req(logits.dtype == torch.float32 and tuple(logits.shape) == (T, E_GLOBAL) and logits.is_contiguous(),
             "logits must be a contiguous float32 [T, 256]")
        _req(q.dtype == torch.float8_e4m3fn and tuple(q.shape) == (T, H) and q.is_contiguous(),
             "q must be a contiguous float8_e4m3fn [T, 7168]")
        _req(scale.dtype == torch.float32 and tuple(scale.shape) == (H // BLOCK, T) and scale.is_contiguous(),
             "scale must be a contiguous float32 [56, T]")
    if T == 0:
        return logits, q, scale
    x, g = _contig(hidden_bf16), _contig(gate_weight)
    with torch.cuda.device(dev):
        code = _lib.load().moe_fp8_router_quantize(x.data_ptr(), g.data_ptr(), T, logits.data_ptr(), q.data_ptr(),
                                                   scale.data_ptr(), _stream(dev))
    _lib.check(code, "moe_fp8_router_quantize")
    return logits, q, scale


@torch.no_grad()
def dispatch(topk_ids, topk_w, tok_pair, local_expert_offset):
    """Dispatch stage: returns (header int32 [128], perm_tok int32 [8T], perm_w fp32 [8T], tok_pair).

    ``header`` holds counts[32], seg_start[33], n_active, active[32]. ``tok_pair``
    (from ``route``) is updated in place with each local pair's index.
    """
    _on_gpu(topk_ids, "topk_ids")
    T = topk_ids.shape[0]
    dev = topk_ids.device
    header = torch.zeros(_header_words(T), dtype=torch.int32, device=dev)
    perm_tok = torch.full((max(1, TOP_K * T),), -1, dtype=torch.int32, device=dev)
    perm_w = torch.zeros((max(1, TOP_K * T),), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        code = _lib.load().moe_fp8_dispatch(topk_ids.data_ptr() if T else None,
                                            topk_w.data_ptr() if T else None, T, int(local_expert_offset),
                                            header.data_ptr(), header.numel(), perm_tok.data_ptr(),
                                            perm_w.data_ptr(), tok_pair.data_ptr() if T else header.data_ptr(),
                                            _stream(dev))
    _lib.check(code, "moe_fp8_dispatch")
    return header[:_lib.MOE_FP8_HEADER_WORDS], perm_tok, perm_w, tok_pair


@torch.no_grad()
def route_dispatch(routing_logits, routing_bias, local_expert_offset, routed_scaling_factor, shape=SHAPE_AUTO):
    """Routing + dispatch exactly as ``run_shape(shape, ...)`` runs them.

    Returns (topk_ids int32 [T, 8], topk_w fp32 [T, 8], header int32 [128],
    perm_tok int32 [8T], perm_w fp32 [8T], tok_pair int32 [T, 8]).
    """
    _on_gpu(routing_logits, "routing_logits")
    _req(routing_logits.dtype == torch.float32 and routing_logits.dim() == 2
         and routing_logits.shape[1] == E_GLOBAL, "routing_logits must be float32 [T, 256]")
    _req(routing_bias.dtype == torch.bfloat16 and routing_bias.numel() == E_GLOBAL, "routing_bias must be bf16 [256]")
    T = routing_logits.shape[0]
    dev = routing_logits.device
    ids = torch.empty((T, TOP_K), dtype=torch.int32, device=dev)
    w = torch.empty((T, TOP_K), dtype=torch.float32, device=dev)
    header = torch.zeros(_header_words(T), dtype=torch.int32, device=dev)
    perm_tok = torch.full((max(1, TOP_K * T),), -1, dtype=torch.int32, device=dev)
    perm_w = torch.zeros((max(1, TOP_K * T),), dtype=torch.float32, device=dev)
    pair = torch.full((T, TOP_K), -7, dtype=torch.int32, device=dev)
    if T == 0:
        return ids, w, header[:_lib.MOE_FP8_HEADER_WORDS], perm_tok, perm_w, pair
    lg, b = _contig(routing_logits), _contig(routing_bias.reshape(-1))
    with torch.cuda.device(dev):
        code = _lib.load().moe_fp8_route_dispatch(int(shape), lg.data_ptr(), b.data_ptr(), T, int(local_expert_offset),
                                                  float(routed_scaling_factor), ids.data_ptr(), w.data_ptr(),
                                                  header.data_ptr(), header.numel(), perm_tok.data_ptr(),
                                                  perm_w.data_ptr(), pair.data_ptr(), _stream(dev))
    _lib.check(code, "moe_fp8_route_dispatch")
    return ids, w, header[:_lib.MOE_FP8_HEADER_WORDS], perm_tok, perm_w, pair
