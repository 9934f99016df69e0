"""Gated-delta scan ops on MI355X, behind the reference's op signatures.

Reference call sites this module replaces:

* ``gated_delta_kernel(q, k, v, g, beta, state, mask)`` -> ``(out, state)``
  (mlx_lm 0.31.2, called at dflash_mlx/custom_qwen35_model.py:457-466 and
  :365-374).  ``gated_delta_verify`` adds the third output, the per-token state
  tape, and is registered as the torch op ``dflash::gated_delta_verify``.
* ``advance_gated_delta_states(initial_states, keys, values, g, beta)``
  (custom_qwen35_model.py:97-139): the state-only replay.
* the rollback gathers of ``rollback_linear_caches``
  (custom_qwen35_model.py:1029-1074): ``tape_select`` and ``conv_rollback``.

Every op runs a hand-written gfx950 kernel of libdflash_gfx950.so on torch's
current stream; allocation stays with torch's caching allocator.  Inputs that
are not on a ROCm device, or shapes the kernels do not support, raise.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _lib

_STATE_DTYPE = torch.float32


def _require_device(name: str, t: torch.Tensor, device: torch.device | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a ROCm device (got {t.device}); there is no CPU path")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def _inner_contig(name: str, t: torch.Tensor) -> torch.Tensor:
    """Innermost dim must be unit-stride; other strides are passed through."""
    if t.stride(-1) != 1:
        t = t.contiguous()
    return t


def _check_scan_inputs(q, k, v, g, beta, state):
    if k.dim() != 4 or v.dim() != 4:
        raise ValueError("k must be [B,T,Hk,Dk] and v [B,T,Hv,Dv]")
    B, T, Hk, Dk = k.shape
    Bv, Tv, Hv, Dv = v.shape
    if (Bv, Tv) != (B, T):
        raise ValueError(f"v batch/time {tuple(v.shape[:2])} != k {tuple(k.shape[:2])}")
    if q is not None and tuple(q.shape) != tuple(k.shape):
        raise ValueError(f"q shape {tuple(q.shape)} != k shape {tuple(k.shape)}")
    if tuple(g.shape) != (B, T, Hv) or tuple(beta.shape) != (B, T, Hv):
        raise ValueError(f"g and beta must be [B,T,Hv] = {(B, T, Hv)}")
    if tuple(state.shape) != (B, Hv, Dv, Dk):
        raise ValueError(f"state must be [B,Hv,Dv,Dk] = {(B, Hv, Dv, Dk)}, got {tuple(state.shape)}")
    if Hv % Hk != 0:
        raise ValueError(f"Hv={Hv} must be a multiple of Hk={Hk}")
    for name, t in (("k", k), ("v", v)) + ((("q", q),) if q is not None else ()):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    dev = k.device
    for name, t in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta), ("state", state)):
        if t is not None:
            _require_device(name, t, dev)
    return B, T, Hk, Hv, Dk, Dv


def _prep(q, k, v, g, beta, state):
    q = _inner_contig("q", q) if q is not None else None
    k = _inner_contig("k", k)
    v = _inner_contig("v", v)
    # g comes from compute_g in fp32; beta is sigmoid(b) and may be bf16 in a
    # bf16 model: both are read as fp32 by the kernel.
    g = _inner_contig("g", g.to(torch.float32))
    beta = _inner_contig("beta", beta.to(torch.float32))
    if state.dtype != _STATE_DTYPE:
        raise TypeError(f"state must be float32 (the fp32 recurrent state), got {state.dtype}")
    state = state.contiguous()
    qs = q.stride()[:3] if q is not None else (0, 0, 0)
    strides = (ctypes.c_int64 * 13)(
        *qs, *k.stride()[:3], *v.stride()[:3], *g.stride()[:2], *beta.stride()[:2])
    return q, k, v, g, beta, state, strides


def _scan(q, k, v, g, beta, state, want_out: bool, want_tape: bool, lengths=None):
    B, T, Hk, Hv, Dk, Dv = _check_scan_inputs(q if want_out else None, k, v, g, beta, state)
    q, k, v, g, beta, state, strides = _prep(q if want_out else None, k, v, g, beta, state)
    dev = k.device
    out = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device=dev) if want_out else None
    final = torch.empty((B, Hv, Dv, Dk), dtype=_STATE_DTYPE, device=dev)
    tape = torch.empty((T, B, Hv, Dv, Dk), dtype=_STATE_DTYPE, device=dev) if want_tape else None
    if lengths is not None:
        _require_device("lengths", lengths, dev)
        lengths = lengths.to(torch.int32).contiguous()
    _lib.call(
        "dflash_gdn_verify_scan",
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta), _lib.ptr(state),
        _lib.ptr(out), _lib.ptr(final), _lib.ptr(tape), _lib.ptr(lengths),
        B, T, Hk, Hv, Dk, Dv, strides, _lib.stream_handle(dev),
    )
    return out, final, tape


@torch.library.custom_op("dflash::gated_delta_verify", mutates_args=())
def gated_delta_verify(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    state: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(q, k, v, g, beta, state) -> (out, final_state, state_tape).

    q, k: [B,T,Hk,Dk] bf16; v: [B,T,Hv,Dv] bf16; g, beta: [B,T,Hv];
    state: [B,Hv,Dv,Dk] fp32.  out: [B,T,Hv,Dv] bf16; final_state: fp32
    [B,Hv,Dv,Dk]; state_tape: fp32 [T,B,Hv,Dv,Dk] with state_tape[t] the state
    after token t (state_tape[T-1] == final_state)."""
    out, final, tape = _scan(q, k, v, g, beta, state, want_out=True, want_tape=True)
    return out, final, tape


@gated_delta_verify.register_fake
def _(q, k, v, g, beta, state):
    B, T, Hk, Dk = k.shape
    Hv, Dv = v.shape[2], v.shape[3]
    return (
        q.new_empty((B, T, Hv, Dv), dtype=torch.bfloat16),
        q.new_empty((B, Hv, Dv, Dk), dtype=_STATE_DTYPE),
        q.new_empty((T, B, Hv, Dv, Dk), dtype=_STATE_DTYPE),
    )


def gated_delta_kernel(q, k, v, g, beta, state, mask=None):
    """Drop-in for mlx_lm's gated_delta_kernel: returns (out, final_state)
    without a tape (the reference's forward, custom_qwen35_model.py:457-466).

    ``mask`` (bool or 0/1 [B, T], the reference's SSM mask of left-padded
    batches, built by create_ssm_mask at custom_qwen35_model.py:968-969):
    a masked token leaves the recurrent state unchanged and its output is
    zero.  It runs as the same scan with g = 1 and beta = 0 at masked
    tokens, which carries the state through bit for bit (S * 1 + k * 0)."""
    if mask is not None:
        B, T = k.shape[0], k.shape[1]
        m = torch.as_tensor(mask, device=k.device)
        if m.dim() != 2 or tuple(m.shape) != (B, T):
            raise ValueError(f"mask must be [B, T] = [{B}, {T}], got {tuple(m.shape)}")
        m = m.to(torch.bool)
        g = torch.where(m[..., None], g.to(torch.float32), 1.0)
        beta = torch.where(m[..., None], beta.to(torch.float32), 0.0)
        out, final, _ = _scan(q, k, v, g, beta, state, want_out=True, want_tape=False)
        return out * m[..., None, None].to(out.dtype), final
    out, final, _ = _scan(q, k, v, g, beta, state, want_out=True, want_tape=False)
    return out, final


def chunked_prefill_workspace_bytes(B: int, T: int, Hv: int, Dk: int = 128, Dv: int = 128) -> int:
    return int(_lib.load().dflash_gdn_chunked_prefill_workspace_bytes(B, T, Hv, Dk, Dv))


def gated_delta_prefill(q, k, v, g, beta, state, workspace: torch.Tensor | None = None):
    """Prompt prefill of one gated-delta layer: (out, final_state), chunked form.

    The recurrence of ``gated_delta_kernel`` evaluated 64 tokens at a time on
    the matrix cores (the prompt pass gated_delta_update,
    custom_qwen35_model.py:790-801).  Agrees with the sequential scan to fp32
    rounding.  ``workspace``: optional uint8 device buffer of at least
    ``chunked_prefill_workspace_bytes(B, T, Hv)`` bytes (else allocated)."""
    B, T, Hk, Hv, Dk, Dv = _check_scan_inputs(q, k, v, g, beta, state)
    q, k, v, g, beta, state, strides = _prep(q, k, v, g, beta, state)
    dev = k.device
    out = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device=dev)
    final = torch.empty((B, Hv, Dv, Dk), dtype=_STATE_DTYPE, device=dev)
    if B == 0 or T == 0:
        final.copy_(state)
        return out, final
    need = chunked_prefill_workspace_bytes(B, T, Hv, Dk, Dv)
    if need == 0:
        raise ValueError(f"chunked prefill supports Dk == Dv == 128 (got Dk={Dk}, Dv={Dv})")
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} bytes, "
                         f"{need} needed")
    _require_device("workspace", workspace, dev)
    _lib.call(
        "dflash_gdn_chunked_prefill",
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta), state.data_ptr(),
        out.data_ptr(), final.data_ptr(), B, T, Hk, Hv, Dk, Dv, strides,
        workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        _lib.stream_handle(dev),
    )
    return out, final


def gated_delta_verify_rollback(q, k, v, g, beta, state, prev_tape, prev_accepted,
                                accepted_period: int | None = None, tape_out=None):
    """Verify scan with the previous step's rollback fused into the state load.

    For sequence b with a = prev_accepted[b % accepted_period] (device int32),
    the block starts from prev_tape[a-1, b] (a >= 1) or state[b] (a == 0);
    ``state`` is updated in place to that rolled-back initial state.  Returns
    (out, tape).  ``tape_out`` may be ``prev_tape`` itself (in-place reuse).
    The device-side counterpart of rollback_linear_caches + the next scan
    (custom_qwen35_model.py:1029-1074, :457-466), with no host sync."""
    B, T, Hk, Hv, Dk, Dv = _check_scan_inputs(q, k, v, g, beta, state)
    if state.dtype != _STATE_DTYPE or not state.is_contiguous():
        raise ValueError("state must be a contiguous float32 buffer (it is updated in place)")
    q, k, v, g, beta, _, strides = _prep(q, k, v, g, beta, state)
    dev = k.device
    _require_device("prev_tape", prev_tape, dev)
    _require_device("prev_accepted", prev_accepted, dev)
    if prev_tape.dtype != _STATE_DTYPE or not prev_tape.is_contiguous():
        raise ValueError("prev_tape must be a contiguous float32 tape")
    if tuple(prev_tape.shape[1:]) != (B, Hv, Dv, Dk):
        raise ValueError(f"prev_tape must be [T', B, Hv, Dv, Dk], got {tuple(prev_tape.shape)}")
    acc = prev_accepted.to(torch.int32).reshape(-1).contiguous()
    period = acc.numel() if accepted_period is None else int(accepted_period)
    if period <= 0 or acc.numel() < period or B % period != 0:
        raise ValueError(f"accepted_period {period} must divide the batch {B} and fit prev_accepted")
    out = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device=dev)
    if tape_out is None:
        tape_out = torch.empty((T, B, Hv, Dv, Dk), dtype=_STATE_DTYPE, device=dev)
    elif tuple(tape_out.shape) != (T, B, Hv, Dv, Dk) or not tape_out.is_contiguous():
        raise ValueError("tape_out must be a contiguous [T, B, Hv, Dv, Dk] float32 tensor")
    _lib.call(
        "dflash_gdn_verify_scan_rollback",
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta), state.data_ptr(),
        prev_tape.data_ptr(), acc.data_ptr(), prev_tape.shape[0], period,
        out.data_ptr(), None, tape_out.data_ptr(), B, T, Hk, Hv, Dk, Dv, strides,
        _lib.stream_handle(dev),
    )
    return out, tape_out


def advance_gated_delta_states(initial_states, keys, values, g, beta, lengths=None):
    """State after replaying keys.shape[1] tokens (or lengths[b] per sequence).

    Mirrors custom_qwen35_model.py:97-139: keys may already be repeated to the
    Hv value heads (as the reference passes them) or carry Hk < Hv heads."""
    if initial_states.dtype != _STATE_DTYPE:
        raise TypeError("initial_states must be float32")
    _, final, _ = _scan(None, keys, values, g, beta, initial_states, want_out=False,
                        want_tape=False, lengths=lengths)
    return final


def _accepted_tensor(accepted, B: int, device: torch.device) -> torch.Tensor:
    if isinstance(accepted, torch.Tensor):
        _require_device("accepted", accepted, device)
        a = accepted.to(torch.int32).reshape(-1).contiguous()
    else:
        vals = [int(accepted)] * B if isinstance(accepted, int) else [int(x) for x in accepted]
        a = torch.tensor(vals, dtype=torch.int32).to(device)
    if a.numel() != B:
        raise ValueError(f"accepted has {a.numel()} entries, expected {B}")
    return a


def tape_select(
    tapes: Sequence[torch.Tensor],
    states_in: Sequence[torch.Tensor],
    accepted,
    states_out: Sequence[torch.Tensor] | None = None,
) -> list[torch.Tensor]:
    """Per layer l and sequence b: state after ``accepted[b]`` tokens,
    i.e. tapes[l][a-1, b] (a >= 1) or states_in[l][b] (a == 0).

    ``accepted`` is an int, a host list or a device int tensor [B] (read on the
    device: no synchronisation).  states_out may be states_in (in place)."""
    if len(tapes) != len(states_in):
        raise ValueError("tapes and states_in differ in length")
    if not tapes:
        return []
    T, B = tapes[0].shape[:2]
    S = states_in[0][0].numel() if B else 0
    dev = tapes[0].device
    tstride = tapes[0].stride(0)
    for l, (tp, st) in enumerate(zip(tapes, states_in)):
        _require_device(f"tapes[{l}]", tp, dev)
        _require_device(f"states_in[{l}]", st, dev)
        if tp.dtype != _STATE_DTYPE or st.dtype != _STATE_DTYPE:
            raise TypeError("tapes and states must be float32")
        # Each tape[t] must be a contiguous [B, ...] block; the token stride
        # may be wider (per-layer views of one layer-stacked tape).
        if T > 1 and tp.stride(0) != tstride:
            raise ValueError("all tapes must share one token stride")
        if not st.is_contiguous() or (T > 0 and (not tp[0].is_contiguous() or tstride < B * S)):
            raise ValueError("tape[t] blocks and states must be contiguous")
        if tp.shape[0] != T or tp.shape[1] != B or tuple(tp.shape[1:]) != tuple(st.shape):
            raise ValueError(f"tapes[{l}] {tuple(tp.shape)} does not match states_in[{l}] {tuple(st.shape)}")
    if states_out is None:
        states_out = [torch.empty_like(st) for st in states_in]
    for l, so in enumerate(states_out):
        _require_device(f"states_out[{l}]", so, dev)
        if so.shape != states_in[l].shape or so.dtype != _STATE_DTYPE or not so.is_contiguous():
            raise ValueError(f"states_out[{l}] must match states_in[{l}]")
    a = _accepted_tensor(accepted, B, dev)
    _lib.call(
        "dflash_tape_select",
        _lib.ptr_array(tapes), _lib.ptr_array(states_in), _lib.ptr_array(states_out),
        a.data_ptr(), len(tapes), B, T, S, tstride if T > 0 else 0, _lib.stream_handle(dev),
    )
    return list(states_out)


def conv_rollback(
    conv_in: Sequence[torch.Tensor],
    qkv: Sequence[torch.Tensor],
    accepted,
    conv_out: Sequence[torch.Tensor] | None = None,
) -> list[torch.Tensor]:
    """concat(conv_in[l][b], qkv[l][b, :a_b], axis=0)[-K1:] for every layer l
    and sequence b (custom_qwen35_model.py:1044-1051).  conv_in: [B,K1,C];
    qkv: [B,T,C] (C contiguous).  conv_out may be conv_in (in place)."""
    if len(conv_in) != len(qkv):
        raise ValueError("conv_in and qkv differ in length")
    if not conv_in:
        return []
    B, K1, C = conv_in[0].shape
    T = qkv[0].shape[1]
    dev = conv_in[0].device
    dt = conv_in[0].dtype
    qs = qkv[0].stride()
    for l, (ci, qk) in enumerate(zip(conv_in, qkv)):
        _require_device(f"conv_in[{l}]", ci, dev)
        _require_device(f"qkv[{l}]", qk, dev)
        if ci.shape != (B, K1, C) or not ci.is_contiguous() or ci.dtype != dt:
            raise ValueError(f"conv_in[{l}] must be contiguous [B,K1,C] = {(B, K1, C)} of {dt}")
        if qk.shape != (B, T, C) or qk.dtype != dt or qk.stride(-1) != 1 or qk.stride() != qs:
            raise ValueError(f"qkv[{l}] must be [B,T,C] = {(B, T, C)} of {dt} with shared strides")
    if dt.itemsize not in (2, 4):
        raise TypeError(f"unsupported conv-state dtype {dt}")
    if conv_out is None:
        conv_out = [torch.empty_like(ci) for ci in conv_in]
    for l, co in enumerate(conv_out):
        _require_device(f"conv_out[{l}]", co, dev)
        if co.shape != (B, K1, C) or co.dtype != dt or not co.is_contiguous():
            raise ValueError(f"conv_out[{l}] must match conv_in[{l}]")
    a = _accepted_tensor(accepted, B, dev)
    _lib.call(
        "dflash_conv_rollback",
        _lib.ptr_array(conv_in), _lib.ptr_array(qkv), _lib.ptr_array(conv_out), a.data_ptr(),
        len(conv_in), B, T, K1, C, qs[0], qs[1], dt.itemsize, _lib.stream_handle(dev),
    )
    return list(conv_out)
