"""The decode layer's non-attention ops on the GPU (include/sfa_layer.h) for
torch device tensors: thin checks and ctypes calls into libsfa.so.

They restate build_router_segment / build_expert_segment of the reference
(src/model/engine/engine.cpp:1877-1925, 1945-1986): rms_norm * weight,
mul_mat (+ residual), the softmax top-k routing and the SwiGLU experts.
Weights are row-major [n_out][n_in] (ggml ne = [n_in, n_out]), f32 or f16;
expert stacks are [n_expert][n_out][n_in].
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import SFA_KV_F16, SFA_KV_F32

__all__ = ["rms_norm", "mul_mat_vec", "moe_route", "moe_gate", "moe_norm_gate", "moe_ffn", "weight_type"]


def _stream(stream) -> int:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def weight_type(w: torch.Tensor) -> int:
    try:
        return {torch.float32: SFA_KV_F32, torch.float16: SFA_KV_F16}[w.dtype]
    except KeyError:
        raise ValueError(f"weights must be float32 or float16, not {w.dtype}") from None


def _f32(t: torch.Tensor, what: str) -> None:
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError(f"{what} must be a contiguous float32 tensor")


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, out: torch.Tensor | None = None,
             stream=None) -> torch.Tensor:
    """x [n_rows, n] -> (x / rms) * weight (engine.cpp:1879-1880, 1908-1909)."""
    _f32(x, "x")
    _f32(weight, "weight")
    n_rows, n = x.shape
    assert weight.shape == (n,)
    out = torch.empty_like(x) if out is None else out
    _lib.check(_lib.load().sfa_rms_norm(x.data_ptr(), weight.data_ptr(), out.data_ptr(), n_rows, n,
                                        float(eps), _stream(stream)), "sfa_rms_norm")
    return out


def mul_mat_vec(w: torch.Tensor, x: torch.Tensor, residual: torch.Tensor | None = None,
                out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """x [n_rows, n_in] -> x @ w.T (+ residual) [n_rows, n_out] (ggml_mul_mat(w, x))."""
    _f32(x, "x")
    assert w.is_contiguous() and w.dim() == 2 and w.shape[1] == x.shape[1]
    n_rows, n_in = x.shape
    n_out = w.shape[0]
    if residual is not None:
        _f32(residual, "residual")
        assert residual.shape == (n_rows, n_out)
    out = torch.empty((n_rows, n_out), dtype=torch.float32, device=x.device) if out is None else out
    _lib.check(_lib.load().sfa_mul_mat_vec(w.data_ptr(), weight_type(w), x.data_ptr(),
                                           None if residual is None else residual.data_ptr(),
                                           out.data_ptr(), n_rows, n_in, n_out, _stream(stream)),
               "sfa_mul_mat_vec")
    return out


def moe_route(logits: torch.Tensor, n_used: int, ids: torch.Tensor | None = None,
              weights: torch.Tensor | None = None, stream=None):
    """logits [n_rows, n_expert] -> (ids int32, weights f32) [n_rows, n_used]."""
    _f32(logits, "logits")
    n_rows, n_expert = logits.shape
    if ids is None:
        ids = torch.empty((n_rows, n_used), dtype=torch.int32, device=logits.device)
    if weights is None:
        weights = torch.empty((n_rows, n_used), dtype=torch.float32, device=logits.device)
    _lib.check(_lib.load().sfa_moe_route(logits.data_ptr(), n_rows, n_expert, n_used, ids.data_ptr(),
                                         weights.data_ptr(), _stream(stream)), "sfa_moe_route")
    return ids, weights


def moe_gate(gate_inp: torch.Tensor, x: torch.Tensor, n_used: int, ids: torch.Tensor | None = None,
             weights: torch.Tensor | None = None, stream=None):
    """The router product and the routing in one launch: x [n_rows, n_embd],
    gate_inp [n_expert, n_embd] -> (ids int32, weights f32) [n_rows, n_used]."""
    _f32(x, "x")
    n_rows, n_embd = x.shape
    n_expert = gate_inp.shape[0]
    assert gate_inp.is_contiguous() and gate_inp.shape == (n_expert, n_embd)
    if ids is None:
        ids = torch.empty((n_rows, n_used), dtype=torch.int32, device=x.device)
    if weights is None:
        weights = torch.empty((n_rows, n_used), dtype=torch.float32, device=x.device)
    _lib.check(_lib.load().sfa_moe_gate(gate_inp.data_ptr(), weight_type(gate_inp), x.data_ptr(), n_rows, n_embd,
                                        n_expert, n_used, ids.data_ptr(), weights.data_ptr(), _stream(stream)),
               "sfa_moe_gate")
    return ids, weights


def moe_norm_gate(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, gate_inp: torch.Tensor, n_used: int,
                  out: torch.Tensor | None = None, ids: torch.Tensor | None = None,
                  weights: torch.Tensor | None = None, stream=None):
    """rms_norm(x) * norm_weight and the routing of the normed rows in one
    launch: -> (y f32 [n_rows, n_embd], ids int32, weights f32 [n_rows, n_used]),
    equal bit for bit to rms_norm followed by moe_gate."""
    _f32(x, "x")
    _f32(norm_weight, "norm_weight")
    n_rows, n_embd = x.shape
    n_expert = gate_inp.shape[0]
    assert gate_inp.is_contiguous() and gate_inp.shape == (n_expert, n_embd)
    assert norm_weight.shape == (n_embd,)
    if out is None:
        out = torch.empty_like(x)
    if ids is None:
        ids = torch.empty((n_rows, n_used), dtype=torch.int32, device=x.device)
    if weights is None:
        weights = torch.empty((n_rows, n_used), dtype=torch.float32, device=x.device)
    _lib.check(_lib.load().sfa_moe_norm_gate(x.data_ptr(), norm_weight.data_ptr(), float(eps), gate_inp.data_ptr(),
                                             weight_type(gate_inp), n_rows, n_embd, n_expert, n_used,
                                             out.data_ptr(), ids.data_ptr(), weights.data_ptr(), _stream(stream)),
               "sfa_moe_norm_gate")
    return out, ids, weights


def moe_ffn(x: torch.Tensor, residual: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
            gate_exps: torch.Tensor, up_exps: torch.Tensor, down_exps: torch.Tensor,
            out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
            stream=None) -> torch.Tensor:
    """The expert segment: x, residual [n_rows, n_embd]; ids / weights
    [n_rows, n_used]; gate/up [n_expert, n_ff, n_embd], down [n_expert, n_embd, n_ff]."""
    _f32(x, "x")
    _f32(residual, "residual")
    n_rows, n_embd = x.shape
    n_expert, n_ff, _ = gate_exps.shape
    n_used = ids.shape[1]
    assert gate_exps.shape == up_exps.shape == (n_expert, n_ff, n_embd)
    assert down_exps.shape == (n_expert, n_embd, n_ff)
    assert gate_exps.dtype == up_exps.dtype == down_exps.dtype
    assert ids.dtype == torch.int32 and ids.is_contiguous() and weights.is_contiguous()
    lib = _lib.load()
    need = lib.sfa_moe_workspace_bytes(n_rows, n_used, n_ff)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    out = torch.empty_like(x) if out is None else out
    _lib.check(lib.sfa_moe_ffn(x.data_ptr(), residual.data_ptr(), ids.data_ptr(), weights.data_ptr(),
                               gate_exps.data_ptr(), up_exps.data_ptr(), down_exps.data_ptr(),
                               weight_type(gate_exps), n_rows, n_embd, n_ff, n_expert, n_used,
                               workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                               out.data_ptr(), _stream(stream)), "sfa_moe_ffn")
    return out
