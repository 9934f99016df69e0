"""Allocation-free verify step for serving loops.

``VerifyStepRunner`` owns every device buffer of one verify step at fixed
shapes and drives the C ABI directly (no torch op dispatch, no per-step
allocation), in the order of the reference's verify_block_parallel_replay
(dflash_mlx/runtime.py:117-163) with the rollback moved onto the device:

  1. gated-delta scan of all linear layers' inputs, writing out, the final
     state and the per-token state tape       (dflash_gdn_verify_scan; in the
     fused form with small logits the accept's argmax runs in the same
     launch)
  2. greedy accept on the verify logits       (dflash_greedy_accept): the
     block's drafts block[1:] against the posterior rows 0..T-2, bonus =
     posterior[matched] (runtime.py:145-147), then keep = matched + 1
     (accepted_inputs, :146; dflash_commit_accept)
  3. recurrent-state rollback by tape gather  (dflash_tape_select, keep)
  4. conv-window rollback                     (dflash_conv_rollback, keep)

The keep count produced by step 2 feeds steps 3-4 on the device, so a step
needs no host synchronisation.  Layers are stacked as batch entries of
one scan launch (batch index = layer * B + b); layer l's tape is the view
tape[:, l*B:(l+1)*B] whose token stride is L*B*S.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib


# The fused step runs the accept's argmax as extra workgroups of the scan's
# launch while the verify logits are at most this many bytes: there a launch
# of its own would be bound by the ~5 us launch floor rather than by reading
# the logits (32 MiB at HBM speed), and the extra workgroups hide it.  Larger
# logits get their own launch after the scan: workgroups sharing CUs with the
# scan's stretch its per-token chain by more than that launch costs.
ARGMAX_IN_SCAN_MAX_BYTES = 32 << 20


@dataclass(frozen=True)
class StepShape:
    L: int        # gated-delta layers in the step
    B: int        # sequences
    T: int        # verify block length
    Hk: int
    Hv: int
    Dk: int
    Dv: int
    V: int        # vocabulary of the verify logits
    conv_dim: int = 0   # 0: no conv-window rollback
    K1: int = 3         # conv kernel size - 1

    def scan_bytes(self) -> int:
        Bt, T = self.L * self.B, self.T
        qkvo = 2 * Bt * T * (2 * self.Hk * self.Dk + 2 * self.Hv * self.Dv)
        gb = 8 * Bt * T * self.Hv
        return qkvo + gb + 4 * Bt * self.Hv * self.Dv * self.Dk * (T + 2)

    def accept_bytes(self, logit_bytes: int = 4) -> int:
        return logit_bytes * self.B * self.T * self.V + 4 * self.B * self.T

    def fuse_argmax(self) -> bool:
        """Whether the fused step runs the accept's argmax inside the scan's
        launch (conv windows present and logits within ARGMAX_IN_SCAN_MAX_BYTES)."""
        return bool(self.conv_dim) and 4 * self.B * self.T * self.V <= ARGMAX_IN_SCAN_MAX_BYTES

    def rollback_bytes(self) -> int:
        """Upper bound (every sequence accepts >= 1 token): state read + write,
        conv window read + write."""
        st = 2 * 4 * self.L * self.B * self.Hv * self.Dv * self.Dk
        cv = 2 * 2 * self.L * self.B * self.K1 * self.conv_dim
        return st + cv


class VerifyStepRunner:
    """Holds the step's device buffers; ``run()`` enqueues one verify step on
    torch's current stream.  Inputs are written into the ``q, k, v, g, beta,
    state, logits, block, conv_in, qkv`` buffers by the caller (``block``:
    the verify block, the last accepted token then T-1 drafts)."""

    def __init__(self, shape: StepShape, device: torch.device):
        s = shape
        self.shape = s
        self.device = device
        Bt = s.L * s.B
        bf, f32, i32 = torch.bfloat16, torch.float32, torch.int32
        # Inputs are written by the caller and outputs by the kernels, so the
        # buffers start uninitialised; only `keep` must start at zero (the
        # first fused step then starts every sequence from `state`).
        z = lambda *shp, dt: torch.empty(shp, dtype=dt, device=device)
        self.q = z(Bt, s.T, s.Hk, s.Dk, dt=bf)
        self.k = z(Bt, s.T, s.Hk, s.Dk, dt=bf)
        self.v = z(Bt, s.T, s.Hv, s.Dv, dt=bf)
        self.g = z(Bt, s.T, s.Hv, dt=f32)
        self.beta = z(Bt, s.T, s.Hv, dt=f32)
        self.state = z(Bt, s.Hv, s.Dv, s.Dk, dt=f32)
        self.out = z(Bt, s.T, s.Hv, s.Dv, dt=bf)
        self.final = z(Bt, s.Hv, s.Dv, s.Dk, dt=f32)
        self.tape = z(s.T, Bt, s.Hv, s.Dv, s.Dk, dt=f32)
        self.new_state = z(Bt, s.Hv, s.Dv, s.Dk, dt=f32)
        self.logits = z(s.B, s.T, s.V, dt=f32)
        self.block = z(s.B, s.T, dt=i32)  # the verify block: last token, then T-1 drafts
        self.posterior = z(s.B, s.T, dt=i32)
        self.matched = torch.zeros(s.B, dtype=i32, device=device)
        self.keep = torch.zeros(s.B, dtype=i32, device=device)  # accepted_inputs = matched + 1
        self.bonus = z(s.B, dt=i32)
        self.argmax_in_scan = s.fuse_argmax()
        lib = _lib.load()
        ws = int(lib.dflash_greedy_accept_workspace_bytes(s.B, s.T, s.V))
        self.workspace = z(max(ws, 8), dt=torch.uint8)
        if s.conv_dim:
            self.conv_in = [z(s.B, s.K1, s.conv_dim, dt=bf) for _ in range(s.L)]
            self.qkv = [z(s.B, s.T, s.conv_dim, dt=bf) for _ in range(s.L)]
            self.conv_out = [z(s.B, s.K1, s.conv_dim, dt=bf) for _ in range(s.L)]
        self._build_args()

    def _build_args(self) -> None:
        s = self.shape
        Bt = s.L * s.B
        S = s.Hv * s.Dv * s.Dk
        self._scan_args = (
            self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.g.data_ptr(),
            self.beta.data_ptr(), self.state.data_ptr(), self.out.data_ptr(),
            self.final.data_ptr(), self.tape.data_ptr(), None,
            Bt, s.T, s.Hk, s.Hv, s.Dk, s.Dv, None,
        )
        # Fused form: the scan starts each sequence from the previous step's
        # tape at its keep count (self.keep), updating self.state in place, and
        # rewrites the same tape buffer; the final state is tape[T-1].
        self._scan_rb_args = (
            self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.g.data_ptr(),
            self.beta.data_ptr(), self.state.data_ptr(), self.tape.data_ptr(),
            self.keep.data_ptr(), s.T, s.B, self.out.data_ptr(), None,
            self.tape.data_ptr(), Bt, s.T, s.Hk, s.Hv, s.Dk, s.Dv, None,
        )
        # drafts = block[1:] (row stride T, T-1 of them) against all T
        # posterior rows: the bonus may come from row T-1
        self._accept_args = (
            self.logits.data_ptr(), _lib.DFLASH_DTYPE_F32, s.T * s.V, s.V,
            self.block.data_ptr() + 4, s.T, s.T - 1, self.posterior.data_ptr(),
            self.matched.data_ptr(), self.bonus.data_ptr(), s.B, s.T, s.V,
            self.workspace.data_ptr(), self.workspace.numel(),
        )
        self._commit_args = (self.matched.data_ptr(), self.keep.data_ptr(), None, s.B, s.T)
        esz = 4
        tapes = (ctypes.c_void_p * s.L)(*[self.tape.data_ptr() + l * s.B * S * esz for l in range(s.L)])
        sins = (ctypes.c_void_p * s.L)(*[self.state.data_ptr() + l * s.B * S * esz for l in range(s.L)])
        souts = (ctypes.c_void_p * s.L)(*[self.new_state.data_ptr() + l * s.B * S * esz
                                          for l in range(s.L)])
        self._tape_args = (tapes, sins, souts, self.keep.data_ptr(), s.L, s.B, s.T, S, Bt * S)
        if s.conv_dim:
            cins = _lib.ptr_array(self.conv_in)
            qkvs = _lib.ptr_array(self.qkv)
            couts = _lib.ptr_array(self.conv_out)
            self._conv_args = (cins, qkvs, couts, self.keep.data_ptr(), s.L, s.B, s.T, s.K1,
                               s.conv_dim, s.T * s.conv_dim, s.conv_dim, 2)
            # accept + conv rollback in two launches (finalize inside the copy),
            # which also writes keep = matched + 1 for the next scan
            self._accept_conv_args = self._accept_args + (
                cins, qkvs, couts, 1, self.keep.data_ptr(), s.L, s.T, s.K1, s.conv_dim,
                s.T * s.conv_dim, s.conv_dim, 2)
            # the same with the argmax already run by the scan's launch
            self._scan_rb_argmax_args = self._scan_rb_args + (
                self.logits.data_ptr(), _lib.DFLASH_DTYPE_F32, s.T * s.V, s.V, s.B, s.T, s.V,
                self.workspace.data_ptr(), self.workspace.numel())
            self._keys_conv_args = (
                self.block.data_ptr() + 4, s.T, s.T - 1, self.posterior.data_ptr(),
                self.matched.data_ptr(), self.bonus.data_ptr(), s.B, s.T, s.V,
                self.workspace.data_ptr(), self.workspace.numel(), cins, qkvs, couts, 1,
                self.keep.data_ptr(), s.L, s.T, s.K1, s.conv_dim, s.T * s.conv_dim, s.conv_dim, 2)
        lib = _lib.load()
        self._accept_conv = lib.dflash_greedy_accept_conv_rollback
        self._scan_rb_argmax = lib.dflash_gdn_verify_scan_rollback_argmax
        self._keys_conv = lib.dflash_accept_keys_conv_rollback
        self._scan = lib.dflash_gdn_verify_scan
        self._scan_rb = lib.dflash_gdn_verify_scan_rollback
        self._accept = lib.dflash_greedy_accept
        self._tsel = lib.dflash_tape_select
        self._conv = lib.dflash_conv_rollback
        self._commit = lib.dflash_commit_accept

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def scan(self, stream: int | None = None) -> None:
        _lib.check("dflash_gdn_verify_scan", self._scan(*self._scan_args, stream or self._stream()))

    def accept(self, stream: int | None = None) -> None:
        """Greedy accept, then keep = matched + 1 (two launches)."""
        st = stream or self._stream()
        _lib.check("dflash_greedy_accept", self._accept(*self._accept_args, st))
        _lib.check("dflash_commit_accept", self._commit(*self._commit_args, st))

    def rollback(self, stream: int | None = None) -> None:
        st = stream or self._stream()
        _lib.check("dflash_tape_select", self._tsel(*self._tape_args, st))
        if self.shape.conv_dim:
            _lib.check("dflash_conv_rollback", self._conv(*self._conv_args, st))

    def scan_rolled(self, stream: int | None = None) -> None:
        _lib.check("dflash_gdn_verify_scan_rollback",
                   self._scan_rb(*self._scan_rb_args, stream or self._stream()))

    def conv_rollback(self, stream: int | None = None) -> None:
        if self.shape.conv_dim:
            _lib.check("dflash_conv_rollback", self._conv(*self._conv_args, stream or self._stream()))

    def accept_conv_rollback(self, stream: int | None = None) -> None:
        """accept() then conv_rollback(), as two launches instead of four (the
        window copy also writes keep)."""
        st = stream or self._stream()
        if not self.shape.conv_dim:
            self.accept(st)
            return
        _lib.check("dflash_greedy_accept_conv_rollback",
                   self._accept_conv(*self._accept_conv_args, st))

    def scan_rolled_argmax(self, stream: int | None = None) -> None:
        """scan_rolled() with the accept's argmax (per-slice keys of the
        verify logits) run by extra workgroups of the same launch."""
        _lib.check("dflash_gdn_verify_scan_rollback_argmax",
                   self._scan_rb_argmax(*self._scan_rb_argmax_args, stream or self._stream()))

    def accept_keys_conv_rollback(self, stream: int | None = None) -> None:
        """The accept's finalize inside the conv-window rollback, from the keys
        scan_rolled_argmax() left in the workspace (one launch)."""
        _lib.check("dflash_accept_keys_conv_rollback",
                   self._keys_conv(*self._keys_conv_args, stream or self._stream()))

    def run(self) -> None:
        """Explicit form: scan (with final state) -> accept -> gather rollback."""
        st = self._stream()
        self.scan(st)
        self.accept(st)
        self.rollback(st)

    def run_fused(self) -> None:
        """Steady-state serving form: scan with the previous step's state
        rollback fused into its load -> accept -> conv-window rollback.  After
        the call, the state after keeping keep[b] = matched[b] + 1 tokens of
        this block is tape[keep[b]-1, b], which the next run_fused() picks up
        on the device.  Start with keep zeroed (the first scan then starts
        from state).  With conv windows and small logits
        (``argmax_in_scan``): two launches, the scan with the accept's argmax,
        then the finalize inside the window copy; otherwise three."""
        st = self._stream()
        if self.argmax_in_scan:
            self.scan_rolled_argmax(st)
            self.accept_keys_conv_rollback(st)
        else:
            self.scan_rolled(st)
            self.accept_conv_rollback(st)

    def rolled_back_state(self) -> torch.Tensor:
        """Materialise the state the next fused step starts from (test helper;
        reads matched on the host)."""
        s = self.shape
        a = self.keep.cpu().repeat(s.L).tolist()
        outs = [self.tape[ai - 1, i] if ai >= 1 else self.state[i] for i, ai in enumerate(a)]
        return torch.stack(outs)
