"""Allocation-free verify step for serving loops.

``VerifyStepRunner`` owns every device buffer of one verify step at fixed
shapes and drives the C ABI directly (no torch op dispatch, no per-step
allocation), in the order of the reference's verify_block_parallel_replay
(dflash_mlx/runtime.py:117-163) with the rollback moved onto the device:

  1. gated-delta scan of all linear layers' inputs, writing out, the final
     state and the per-token state tape       (dflash_gdn_verify_scan)
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


# The fused step runs as one launch (dflash_gdn_verify_step: the accept's
# last argmax workgroup of each sequence finishes the accept and copies the
# conv windows while the scan runs) while the windows are at most this many
# bytes.  One workgroup streams at one CU's rate (~25-30 GB/s): at c0's 48 KB
# the copy hides behind the scan (graph step 10.7-12.4 against 14.5-15.5 us
# in two launches); at c1's 1.2 MB (24 layers of 3 x 8192 bf16) it outlasted
# the scan (194 against 143 us), and with the copy in a launch of its own
# the step launch's finishing argmax workgroups (agent-scope stores and
# counts, fewer of them resident beside the scan) cost more than the launch
# they save (145 against 143 us).  Larger windows keep the two-launch form.
SINGLE_LAUNCH_MAX_CONV_BYTES = 256 << 10

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

    def single_launch(self) -> bool:
        """Whether the fused step runs as one launch (dflash_gdn_verify_step):
        the argmax in the scan's launch, bf16 windows of 16-byte rows within
        SINGLE_LAUNCH_MAX_CONV_BYTES, at most 32 layers, 64 rows, 4 window
        rows."""
        return (self.fuse_argmax() and self.conv_dim % 8 == 0 and self.L <= 32 and self.T <= 64
                and self.K1 <= 4
                and 2 * self.L * self.B * self.K1 * self.conv_dim <= SINGLE_LAUNCH_MAX_CONV_BYTES)

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
    the verify block, the last accepted token then T-1 drafts).

    The keep counts (accepted_inputs = matched + 1) live in two device
    buffers used in turn: a fused step reads the current one (its scan rolls
    each sequence's state back to it) and writes the other, which then
    becomes current (``keep``).  The single-launch form needs that (its
    accept runs while its scan still reads the previous count); the other
    forms follow the same rule so that they can be mixed.  A HIP graph of
    the fused step therefore captures two steps (``run_fused`` twice); it
    holds the buffers that were current at capture, so eager steps between
    its replays come in pairs (``keep`` is the same buffer before and after
    each replay)."""

    def __init__(self, shape: StepShape, device: torch.device, overlap_accept: bool = False):
        """overlap_accept: let the fused step run the accept's argmax inside
        the scan's launch (and, where the windows are small, the whole step in
        one launch).  In a decode the verify logits come out of this block's
        scan (through the later layers and the LM head), so the accept cannot
        start before the scan ends; those forms are schedulable only when the
        logits are given ahead of the scan, as in a synthetic benchmark, and
        are off by default."""
        s = shape
        self.shape = s
        self.device = device
        Bt = s.L * s.B
        bf, f32, i32 = torch.bfloat16, torch.float32, torch.int32
        # Inputs are written by the caller and outputs by the kernels, so the
        # buffers start uninitialised; only the keep counts and the step's
        # arrival counts must start at zero (the first fused step then starts
        # every sequence from `state`).
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
        self._keeps = torch.zeros(2, s.B, dtype=i32, device=device)
        self._pp = 0  # index of the current keep buffer
        self.bonus = z(s.B, dt=i32)
        self.argmax_in_scan = bool(overlap_accept) and s.fuse_argmax()
        lib = _lib.load()
        if s.conv_dim:
            self.conv_in = [z(s.B, s.K1, s.conv_dim, dt=bf) for _ in range(s.L)]
            self.qkv = [z(s.B, s.T, s.conv_dim, dt=bf) for _ in range(s.L)]
            self.conv_out = [z(s.B, s.K1, s.conv_dim, dt=bf) for _ in range(s.L)]
        # With overlap_accept, the whole fused step in one launch
        # (dflash_gdn_verify_step) where its limits allow and pay: argmax in the scan's launch, bf16 windows
        # copied as 16-byte units, at most SINGLE_LAUNCH_MAX_CONV_BYTES of
        # them, 32 layers, 64 rows, 4 window rows.  conv_in_launch False (a
        # form kept for tests and callers with their own measurements): the
        # step launch leaves the windows to a dflash_conv_rollback after it.
        self.conv_in_launch = True
        self.single_launch = bool(overlap_accept) and s.single_launch()
        ws = max(int(lib.dflash_greedy_accept_workspace_bytes(s.B, s.T, s.V)),
                 int(lib.dflash_gdn_verify_step_workspace_bytes(s.B, s.T, s.V)))
        # zeroed: the single-launch step's arrival counts follow the keys
        self.workspace = torch.zeros(max(ws, 8), dtype=torch.uint8, device=device)
        self._build_args()

    @property
    def keep(self) -> torch.Tensor:
        """The current keep counts (int32 [B]): what the next fused step's scan
        rolls back to."""
        return self._keeps[self._pp]

    def _args(self, p: int) -> dict:
        """Launch arguments with keep buffer p current (read by the scans and
        the explicit rollback) and 1 - p the one a fused step writes."""
        s = self.shape
        Bt = s.L * s.B
        S = s.Hv * s.Dv * s.Dk
        kin, kout = self._keeps[p].data_ptr(), self._keeps[1 - p].data_ptr()
        a = {}
        a["scan"] = (
            self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.g.data_ptr(),
            self.beta.data_ptr(), self.state.data_ptr(), self.out.data_ptr(),
            self.final.data_ptr(), self.tape.data_ptr(), None,
            Bt, s.T, s.Hk, s.Hv, s.Dk, s.Dv, None,
        )
        # Fused form: the scan starts each sequence from the previous step's
        # tape at its keep count, updating self.state in place, and rewrites
        # the same tape buffer; the final state is tape[T-1].
        a["scan_rb"] = (
            self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.g.data_ptr(),
            self.beta.data_ptr(), self.state.data_ptr(), self.tape.data_ptr(),
            kin, s.T, s.B, self.out.data_ptr(), None,
            self.tape.data_ptr(), Bt, s.T, s.Hk, s.Hv, s.Dk, s.Dv, None,
        )
        # drafts = block[1:] (row stride T, T-1 of them) against all T
        # posterior rows: the bonus may come from row T-1
        a["accept"] = (
            self.logits.data_ptr(), _lib.DFLASH_DTYPE_F32, s.T * s.V, s.V,
            self.block.data_ptr() + 4, s.T, s.T - 1, self.posterior.data_ptr(),
            self.matched.data_ptr(), self.bonus.data_ptr(), s.B, s.T, s.V,
            self.workspace.data_ptr(), self.workspace.numel(),
        )
        a["commit"] = (self.matched.data_ptr(), kin, None, s.B, s.T)
        esz = 4
        tapes = (ctypes.c_void_p * s.L)(*[self.tape.data_ptr() + l * s.B * S * esz for l in range(s.L)])
        sins = (ctypes.c_void_p * s.L)(*[self.state.data_ptr() + l * s.B * S * esz for l in range(s.L)])
        souts = (ctypes.c_void_p * s.L)(*[self.new_state.data_ptr() + l * s.B * S * esz
                                          for l in range(s.L)])
        a["tape"] = (tapes, sins, souts, kin, s.L, s.B, s.T, S, Bt * S)
        if s.conv_dim:
            cins = _lib.ptr_array(self.conv_in)
            qkvs = _lib.ptr_array(self.qkv)
            couts = _lib.ptr_array(self.conv_out)
            a["conv"] = (cins, qkvs, couts, kin, s.L, s.B, s.T, s.K1,
                         s.conv_dim, s.T * s.conv_dim, s.conv_dim, 2)
            # accept + conv rollback in two launches (finalize inside the copy),
            # which also writes the next keep = matched + 1
            a["accept_conv"] = a["accept"] + (
                cins, qkvs, couts, 1, kout, s.L, s.T, s.K1, s.conv_dim,
                s.T * s.conv_dim, s.conv_dim, 2)
            # the same with the argmax already run by the scan's launch
            a["scan_rb_argmax"] = a["scan_rb"] + (
                self.logits.data_ptr(), _lib.DFLASH_DTYPE_F32, s.T * s.V, s.V, s.B, s.T, s.V,
                self.workspace.data_ptr(), self.workspace.numel())
            a["keys_conv"] = (
                self.block.data_ptr() + 4, s.T, s.T - 1, self.posterior.data_ptr(),
                self.matched.data_ptr(), self.bonus.data_ptr(), s.B, s.T, s.V,
                self.workspace.data_ptr(), self.workspace.numel(), cins, qkvs, couts, 1,
                kout, s.L, s.T, s.K1, s.conv_dim, s.T * s.conv_dim, s.conv_dim, 2)
            # everything in one launch (step), or all but the conv windows (step_noconv)
            step = a["scan_rb"] + (
                self.logits.data_ptr(), _lib.DFLASH_DTYPE_F32, s.T * s.V, s.V, s.B, s.T, s.V,
                self.block.data_ptr() + 4, s.T, s.T - 1, self.posterior.data_ptr(),
                self.matched.data_ptr(), self.bonus.data_ptr(), 1, kout)
            tail = (self.workspace.data_ptr(), self.workspace.numel())
            a["step"] = step + (cins, qkvs, couts, s.L, s.K1, s.conv_dim, s.T * s.conv_dim,
                                s.conv_dim) + tail
            a["step_noconv"] = step + (None, None, None, 0, 0, 0, 0, 0) + tail
            a["_keep_alive"] = (tapes, sins, souts, cins, qkvs, couts)
        return a

    def _build_args(self) -> None:
        self._argsets = [self._args(0), self._args(1)]
        lib = _lib.load()
        self._accept_conv = lib.dflash_greedy_accept_conv_rollback
        self._scan_rb_argmax = lib.dflash_gdn_verify_scan_rollback_argmax
        self._keys_conv = lib.dflash_accept_keys_conv_rollback
        self._step = lib.dflash_gdn_verify_step
        self._scan = lib.dflash_gdn_verify_scan
        self._scan_rb = lib.dflash_gdn_verify_scan_rollback
        self._accept = lib.dflash_greedy_accept
        self._tsel = lib.dflash_tape_select
        self._conv = lib.dflash_conv_rollback
        self._commit = lib.dflash_commit_accept

    def _a(self, name):
        return self._argsets[self._pp][name]

    def _flip(self) -> None:
        """The keep buffer a fused step wrote becomes the current one."""
        self._pp ^= 1

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def scan(self, stream: int | None = None) -> None:
        _lib.check("dflash_gdn_verify_scan", self._scan(*self._a("scan"), stream or self._stream()))

    def accept(self, stream: int | None = None) -> None:
        """Greedy accept, then keep = matched + 1 into the current keep
        buffer (two launches)."""
        st = stream or self._stream()
        _lib.check("dflash_greedy_accept", self._accept(*self._a("accept"), st))
        _lib.check("dflash_commit_accept", self._commit(*self._a("commit"), st))

    def rollback(self, stream: int | None = None) -> None:
        st = stream or self._stream()
        _lib.check("dflash_tape_select", self._tsel(*self._a("tape"), st))
        if self.shape.conv_dim:
            _lib.check("dflash_conv_rollback", self._conv(*self._a("conv"), st))

    def scan_rolled(self, stream: int | None = None) -> None:
        _lib.check("dflash_gdn_verify_scan_rollback",
                   self._scan_rb(*self._a("scan_rb"), stream or self._stream()))

    def conv_rollback(self, stream: int | None = None) -> None:
        if self.shape.conv_dim:
            _lib.check("dflash_conv_rollback", self._conv(*self._a("conv"), stream or self._stream()))

    def accept_conv_rollback(self, stream: int | None = None) -> None:
        """accept() then conv_rollback(), as two launches instead of four (the
        window copy writes the other keep buffer, which becomes current)."""
        st = stream or self._stream()
        if not self.shape.conv_dim:
            self.accept(st)
            return
        _lib.check("dflash_greedy_accept_conv_rollback",
                   self._accept_conv(*self._a("accept_conv"), st))
        self._flip()

    def scan_rolled_argmax(self, stream: int | None = None) -> None:
        """scan_rolled() with the accept's argmax (per-slice keys of the
        verify logits) run by extra workgroups of the same launch."""
        _lib.check("dflash_gdn_verify_scan_rollback_argmax",
                   self._scan_rb_argmax(*self._a("scan_rb_argmax"), stream or self._stream()))

    def accept_keys_conv_rollback(self, stream: int | None = None) -> None:
        """The accept's finalize inside the conv-window rollback, from the keys
        scan_rolled_argmax() left in the workspace (one launch); the keep it
        writes becomes current."""
        _lib.check("dflash_accept_keys_conv_rollback",
                   self._keys_conv(*self._a("keys_conv"), stream or self._stream()))
        self._flip()

    def step_launch(self, stream: int | None = None) -> None:
        """dflash_gdn_verify_step: the scan with the rollback load and the
        accept's argmax workgroups, the last of which finishes the accept
        and, with ``conv_in_launch``, copies the conv windows."""
        name = "step" if self.conv_in_launch else "step_noconv"
        _lib.check("dflash_gdn_verify_step", self._step(*self._a(name), stream or self._stream()))
        self._flip()

    def step_single(self, stream: int | None = None) -> None:
        """The fused step in one launch, or two when the conv windows are
        copied apart (dflash_conv_rollback of the keep the step wrote)."""
        st = stream or self._stream()
        self.step_launch(st)
        if not self.conv_in_launch:
            self.conv_rollback(st)

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
        from state).  Three launches: the scan, then the accept's argmax,
        then its finalize inside the conv-window copy.  With overlap_accept
        (logits given before the scan) and conv windows and small logits:
        one launch (``single_launch``; two with large windows, the copy
        apart), else two with the argmax in the scan's launch
        (``argmax_in_scan``)."""
        st = self._stream()
        if self.single_launch:
            self.step_single(st)
        elif self.argmax_in_scan:
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
