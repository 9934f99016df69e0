"""One gated-delta layer's verify body on MI355X, between its projections.

Mirrors forward_linear_layer_explicit_with_record
(dflash_mlx/custom_qwen35_model.py:409-484) from the projection outputs
(qkv, z, a, b) to the input of out_proj:

  prologue (1 launch): conv1d + silu over concat(conv_state, qkv), q/k
      rms-norm + scale, g = compute_g(A_log, a, dt_bias), beta = sigmoid(b),
      new conv window                                          (:431-450)
  scan     (1 launch): gated delta rule with out, final state and tape (:457-466)
  epilogue (1 launch): RMSNormGated(out, z)                     (:478)

and returns the rollback record the reference builds (:295-304), with the
state tape in place of the k/v/g/beta replay inputs.  The projections, the
out_proj and the MLP are plain GEMMs (hipBLASLt via torch) and stay with the
caller.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from .adapters import make_rollback_record
from .gated_delta import _require_device, gated_delta_verify


# The q/k RMSNorm of the gated-delta layers uses a fixed eps of 1e-6
# (custom_qwen35_model.py:355-356, :446-447, :787-788), independent of
# rms_norm_eps, which sets only the layer norms and the gated norm.
QK_NORM_EPS = 1e-6


@dataclass(frozen=True)
class GatedDeltaConfig:
    """The linear-attention fields of TextModelArgs
    (custom_qwen35_model.py:648-656); defaults are the Qwen3.5-4B shape."""

    linear_num_key_heads: int = 16
    linear_num_value_heads: int = 32
    linear_key_head_dim: int = 128
    linear_value_head_dim: int = 128
    linear_conv_kernel_dim: int = 4
    rms_norm_eps: float = 1e-6

    @property
    def key_dim(self) -> int:
        return self.linear_num_key_heads * self.linear_key_head_dim

    @property
    def value_dim(self) -> int:
        return self.linear_num_value_heads * self.linear_value_head_dim

    @property
    def conv_dim(self) -> int:
        """custom_qwen35_model.py:717: key_dim * 2 + value_dim."""
        return 2 * self.key_dim + self.value_dim


@dataclass
class GatedDeltaWeights:
    """Per-layer parameters used between the projections (GatedDeltaNet,
    custom_qwen35_model.py:718-739): conv1d weight [C, K] (MLX [C, K, 1]
    layout), A_log fp32 [Hv] (kept fp32 by cast_predicate, :1194-1201),
    dt_bias bf16 [Hv], gated-norm weight bf16 [Dv]."""

    conv_weight: torch.Tensor
    A_log: torch.Tensor
    dt_bias: torch.Tensor
    norm_weight: torch.Tensor

    @staticmethod
    def random(cfg: GatedDeltaConfig, device, generator: torch.Generator | None = None):
        """Random-init parameters with the reference's init distributions:
        A = U(0, 16), A_log = log(A); dt_bias = 1; norm weight = 1
        (custom_qwen35_model.py:733-739); conv weight ~ N(0, 1/K)."""
        g = generator
        C, K = cfg.conv_dim, cfg.linear_conv_kernel_dim
        conv = (torch.randn(C, K, generator=g) * (1.0 / K) ** 0.5).to(torch.bfloat16)
        A = torch.rand(cfg.linear_num_value_heads, generator=g) * 16.0
        return GatedDeltaWeights(
            conv_weight=conv.to(device),
            A_log=torch.log(A.clamp_min(1e-4)).to(torch.float32).to(device),
            dt_bias=torch.ones(cfg.linear_num_value_heads, dtype=torch.bfloat16, device=device),
            norm_weight=torch.ones(cfg.linear_value_head_dim, dtype=torch.bfloat16, device=device),
        )


def gdn_prologue(qkv, conv_state, a, b, weights: GatedDeltaWeights, cfg: GatedDeltaConfig):
    """Returns (q, k, v, g, beta, new_conv_state); q/k/v are strided views of
    one [B, T, C] bf16 activation buffer, ready for the scan."""
    _require_device("qkv", qkv, None)
    dev = qkv.device
    B, T, C = qkv.shape
    if C != cfg.conv_dim:
        raise ValueError(f"qkv has {C} channels, the config needs {cfg.conv_dim}")
    K = cfg.linear_conv_kernel_dim
    Hk, Hv = cfg.linear_num_key_heads, cfg.linear_num_value_heads
    Dk, Dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
    for name, t in (("conv_state", conv_state), ("a", a), ("b", b)):
        _require_device(name, t, dev)
    if qkv.dtype != torch.bfloat16 or qkv.stride(-1) != 1:
        raise ValueError("qkv must be bf16 with contiguous channels")
    conv_state = conv_state.contiguous()
    if tuple(conv_state.shape) != (B, K - 1, C) or conv_state.dtype != torch.bfloat16:
        raise ValueError(f"conv_state must be bf16 [B, K-1, C] = {(B, K - 1, C)}")
    a = a.to(torch.bfloat16)
    b = b.to(torch.bfloat16)
    if a.stride(-1) != 1:
        a = a.contiguous()
    if b.stride(-1) != 1:
        b = b.contiguous()
    act = torch.empty((B, T, C), dtype=torch.bfloat16, device=dev)
    g = torch.empty((B, T, Hv), dtype=torch.float32, device=dev)
    beta = torch.empty((B, T, Hv), dtype=torch.float32, device=dev)
    new_state = torch.empty_like(conv_state)
    w = weights
    strides = (ctypes.c_int64 * 4)(a.stride(0), a.stride(1), b.stride(0), b.stride(1))
    _lib.call(
        "dflash_gdn_prologue",
        qkv.data_ptr(), qkv.stride(0), qkv.stride(1), conv_state.data_ptr(),
        w.conv_weight.contiguous().data_ptr(), a.data_ptr(), b.data_ptr(), strides,
        w.A_log.data_ptr(), w.dt_bias.data_ptr(), act.data_ptr(), g.data_ptr(), beta.data_ptr(),
        new_state.data_ptr(), B, T, K, Hk, Hv, Dk, Dv, QK_NORM_EPS, _lib.stream_handle(dev),
    )
    kd = Hk * Dk
    q = act[..., :kd].unflatten(-1, (Hk, Dk))
    k = act[..., kd:2 * kd].unflatten(-1, (Hk, Dk))
    v = act[..., 2 * kd:].unflatten(-1, (Hv, Dv))
    return q, k, v, g, beta, new_state


def gated_rmsnorm(x, z, weight, eps: float = 1e-6):
    """RMSNormGated(x, z) (custom_qwen35_model.py:478): weight * rms_norm(x) *
    silu(z) over the last axis.  x: bf16 [B, T, H, D]; z: bf16 [B, T, H, D]
    (strided views allowed, D contiguous); weight: bf16 [D]."""
    _require_device("x", x, None)
    dev = x.device
    _require_device("z", z, dev)
    x = x.contiguous()
    B, T, H, D = x.shape
    if tuple(z.shape) != (B, T, H, D):
        raise ValueError("z must match x")
    if z.stride(-1) != 1:
        z = z.contiguous()
    y = torch.empty_like(x)
    w = weight.to(torch.bfloat16).contiguous()  # held until the launch is enqueued
    strides = (ctypes.c_int64 * 3)(*z.stride()[:3])
    _lib.call("dflash_gdn_gated_rmsnorm", x.data_ptr(), z.data_ptr(), strides, w.data_ptr(),
              y.data_ptr(), B, T, H, D, float(eps), _lib.stream_handle(dev))
    return y


def gdn_layer_verify(qkv, z, a, b, conv_state, state, weights: GatedDeltaWeights,
                     cfg: GatedDeltaConfig):
    """The layer's verify body from projection outputs to out_proj input.

    qkv [B,T,C], z [B,T,Hv*Dv] (or [B,T,Hv,Dv]), a/b [B,T,Hv] (bf16);
    conv_state [B,K-1,C] bf16; state [B,Hv,Dv,Dk] fp32.  Returns
    (y [B,T,Hv*Dv] bf16, new_conv_state, final_state, tape, rollback_record)."""
    q, k, v, g, beta, new_conv = gdn_prologue(qkv, conv_state, a, b, weights, cfg)
    out, final, tape = gated_delta_verify(q, k, v, g, beta, state)
    B, T = qkv.shape[:2]
    Hv, Dv = cfg.linear_num_value_heads, cfg.linear_value_head_dim
    zz = z.reshape(B, T, Hv, Dv) if z.dim() == 3 else z
    y = gated_rmsnorm(out, zz, weights.norm_weight, cfg.rms_norm_eps)
    record = make_rollback_record(conv_state, state, qkv, tape)
    return y.reshape(B, T, Hv * Dv), new_conv, final, tape, record


def gdn_prologue_verify_rollback(qkv, conv_state, a, b, weights: GatedDeltaWeights,
                                 cfg: GatedDeltaConfig, state, prev_tape, prev_accepted,
                                 accepted_period: int | None = None, tape_out=None):
    """gdn_prologue followed by gated_delta_verify_rollback, in one launch
    (dflash_gdn_prologue_scan_rollback): the scan computes each head's q, k,
    v, g and beta from the projection rows itself.  Same arguments as the two
    calls (the prologue's, then the rollback scan's state / prev_tape /
    prev_accepted / tape_out) and the same (out, tape), bit for bit; the new
    conv window is not produced.  Supported: Dk == 128, T <= 32."""
    from .gated_delta import _STATE_DTYPE

    _require_device("qkv", qkv, None)
    dev = qkv.device
    B, T, C = qkv.shape
    if C != cfg.conv_dim:
        raise ValueError(f"qkv has {C} channels, the config needs {cfg.conv_dim}")
    K = cfg.linear_conv_kernel_dim
    Hk, Hv = cfg.linear_num_key_heads, cfg.linear_num_value_heads
    Dk, Dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
    for name, t in (("conv_state", conv_state), ("a", a), ("b", b), ("state", state),
                    ("prev_tape", prev_tape), ("prev_accepted", prev_accepted)):
        _require_device(name, t, dev)
    if qkv.dtype != torch.bfloat16 or qkv.stride(-1) != 1:
        raise ValueError("qkv must be bf16 with contiguous channels")
    conv_state = conv_state.contiguous()
    if tuple(conv_state.shape) != (B, K - 1, C) or conv_state.dtype != torch.bfloat16:
        raise ValueError(f"conv_state must be bf16 [B, K-1, C] = {(B, K - 1, C)}")
    a = a.to(torch.bfloat16)
    b = b.to(torch.bfloat16)
    if a.stride(-1) != 1:
        a = a.contiguous()
    if b.stride(-1) != 1:
        b = b.contiguous()
    if state.dtype != _STATE_DTYPE or not state.is_contiguous() or \
            tuple(state.shape) != (B, Hv, Dv, Dk):
        raise ValueError("state must be a contiguous float32 [B, Hv, Dv, Dk] buffer "
                         "(it is updated in place)")
    if prev_tape.dtype != _STATE_DTYPE or not prev_tape.is_contiguous() or \
            tuple(prev_tape.shape[1:]) != (B, Hv, Dv, Dk):
        raise ValueError("prev_tape must be a contiguous float32 [T', B, Hv, Dv, Dk] tape")
    acc = prev_accepted.to(torch.int32).reshape(-1).contiguous()
    period = acc.numel() if accepted_period is None else int(accepted_period)
    if period <= 0 or acc.numel() < period or B % period != 0:
        raise ValueError(f"accepted_period {period} must divide the batch {B} and fit prev_accepted")
    out = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device=dev)
    if tape_out is None:
        tape_out = torch.empty((T, B, Hv, Dv, Dk), dtype=_STATE_DTYPE, device=dev)
    elif tuple(tape_out.shape) != (T, B, Hv, Dv, Dk) or not tape_out.is_contiguous():
        raise ValueError("tape_out must be a contiguous [T, B, Hv, Dv, Dk] float32 tensor")
    w = weights
    conv_w = w.conv_weight.contiguous()  # held until the launch is enqueued
    strides = (ctypes.c_int64 * 4)(a.stride(0), a.stride(1), b.stride(0), b.stride(1))
    _lib.call(
        "dflash_gdn_prologue_scan_rollback",
        qkv.data_ptr(), qkv.stride(0), qkv.stride(1), conv_state.data_ptr(), conv_w.data_ptr(),
        a.data_ptr(), b.data_ptr(), strides, w.A_log.data_ptr(), w.dt_bias.data_ptr(),
        state.data_ptr(), prev_tape.data_ptr(), acc.data_ptr(), prev_tape.shape[0], period,
        out.data_ptr(), None, tape_out.data_ptr(), B, T, K, Hk, Hv, Dk, Dv, QK_NORM_EPS,
        _lib.stream_handle(dev),
    )
    return out, tape_out
