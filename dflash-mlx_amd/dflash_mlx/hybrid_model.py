"""The Qwen3.5 hybrid target's verify step on MI355X (config c4).

The reference's target model (Qwen3_5TextModel, dflash_mlx/custom_qwen35_model.py:
849-881, decoder layers :815-846) verifies a 16-token draft block in one
forward: 32 decoder layers, 3 gated-delta ("linear") layers then one gated
full-attention layer, repeated (:818, full_attention_interval = 4), each with
RMSNorm -> mixer -> residual -> RMSNorm -> SwiGLU MLP -> residual; then the
final norm, the LM head, the greedy accept (runtime.py:134-147) and, on a
partial accept, the rollback of the recurrent state, the conv window and the
KV caches (runtime.py:149-160; adapters.py:505-560).

``HybridVerifyRunner`` runs that step on one GPU with every buffer allocated
once:

* GEMMs: the stacked projections of each layer (gated-delta in_proj
  qkv|z|b|a, attention q|k|v, MLP gate|up, and the output projections) on
  this package's verify-sized GEMM (``dflash_gemm_bf16``: the weight
  streamed once against the 16 block rows, split-K where N is small, the
  partial sums folded into the next add + RMSNorm, the MLP gating fused into
  the gate|up projection);
* everything else on this package's gfx950 kernels through the C ABI:
  residual add + RMSNorm, the gated-delta prologue, the scan with the previous
  step's rollback fused into its state load (per-token tape), the gated
  RMSNorm, q/k norm + rotary + KV append, split-K verify attention + gate,
  SwiGLU, the fused LM-head greedy accept, and the commit (keep counts, KV
  lengths, conv windows).

Cache lengths and accept counts stay in device memory and no step reads
anything back to the host, so one step can be captured as a HIP graph and
replayed (``capture_step`` / ``replay``).  The reference-API facade
(``target.HybridTargetModel``) drives the same runner one host-synchronous
step at a time.

Random-init weights (bf16 ~ N(0, std) for every projection, unit norms, the
reference's gated-delta parameter inits) and synthetic caches stand in for a
checkpoint; there is no network here.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from . import _lib
from .gdn_layer import QK_NORM_EPS, GatedDeltaConfig, GatedDeltaWeights


@dataclass(frozen=True)
class HybridConfig:
    """TextModelArgs fields of the verify path (custom_qwen35_model.py:638-697)
    at the config-c4 shape: hidden 2560, 32 layers (3:1), 16 query / 4 KV
    heads of 128, vocab 151936.  intermediate_size is not fixed by the config
    or the reference (its default 14336 is a different model); 9216 is used."""

    hidden_size: int = 2560
    num_hidden_layers: int = 32
    full_attention_interval: int = 4
    intermediate_size: int = 9216
    vocab_size: int = 151936
    num_attention_heads: int = 16
    num_key_value_heads: int = 4
    head_dim: int = 128
    rope_theta: float = 100000.0
    partial_rotary_factor: float = 0.25
    rms_norm_eps: float = 1e-6
    linear: GatedDeltaConfig = field(default_factory=GatedDeltaConfig)

    def is_linear(self, i: int) -> bool:
        """DecoderLayer.is_linear (custom_qwen35_model.py:818)."""
        return (i + 1) % self.full_attention_interval != 0

    @property
    def rot_dims(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)

    @property
    def n_linear(self) -> int:
        return sum(self.is_linear(i) for i in range(self.num_hidden_layers))

    @property
    def n_attention(self) -> int:
        return self.num_hidden_layers - self.n_linear

    @property
    def in_proj_rows(self) -> int:
        """Stacked gated-delta input projections qkv | z | b | a (:726-731)."""
        lc = self.linear
        return lc.conv_dim + lc.value_dim + 2 * lc.linear_num_value_heads

    @property
    def attn_proj_rows(self) -> int:
        """Stacked q (query|gate per head) | k | v projections."""
        return (2 * self.num_attention_heads + 2 * self.num_key_value_heads) * self.head_dim


def _bf16_randn(shape, std, generator, device):
    return (torch.randn(*shape, generator=generator, device=generator.device) * std).to(
        torch.bfloat16).to(device)


@dataclass
class HybridWeights:
    embed: torch.Tensor
    final_norm: torch.Tensor
    lm_head: torch.Tensor
    layers: list
    # The LM head's fragment-tiled copy, made by the first runner that streams
    # it (tile_weight; V % 16 == 0).
    lm_head_tiled: torch.Tensor | None = None

    @staticmethod
    def random(cfg: HybridConfig, device, seed: int = 0, std: float = 0.02,
               on_device: bool = True) -> "HybridWeights":
        """bf16 ~ N(0, std) projections and embeddings, unit RMSNorm weights,
        the reference's gated-delta inits (A = U(0,16), dt_bias = 1, norm 1;
        :733-739).  on_device=False draws on the CPU (reproducible on the host,
        for small test configs); True draws with a device generator."""
        gen = torch.Generator(device=device if on_device else "cpu").manual_seed(seed)
        cpu_gen = torch.Generator().manual_seed(seed + 1)
        H, I = cfg.hidden_size, cfg.intermediate_size
        ones = lambda n: torch.ones(n, dtype=torch.bfloat16, device=device)  # noqa: E731
        layers = []
        for i in range(cfg.num_hidden_layers):
            lw = {"ln_in": ones(H), "ln_post": ones(H),
                  "w_gu": _bf16_randn((2 * I, H), std, gen, device),
                  "w_down": _bf16_randn((H, I), std, gen, device)}
            if cfg.is_linear(i):
                lc = cfg.linear
                lw["w_in"] = _bf16_randn((cfg.in_proj_rows, H), std, gen, device)
                lw["w_out"] = _bf16_randn((H, lc.value_dim), std, gen, device)
                lw["gdn"] = GatedDeltaWeights.random(lc, device, cpu_gen)
            else:
                D = cfg.head_dim
                lw["w_qkv"] = _bf16_randn((cfg.attn_proj_rows, H), std, gen, device)
                lw["w_o"] = _bf16_randn((H, cfg.num_attention_heads * D), std, gen, device)
                lw["q_norm"] = ones(D)
                lw["k_norm"] = ones(D)
            layers.append(lw)
        return HybridWeights(
            embed=_bf16_randn((cfg.vocab_size, H), std, gen, device),
            final_norm=ones(H),
            lm_head=_bf16_randn((cfg.vocab_size, H), std, gen, device),
            layers=layers)


def check_cache_lengths(lens, B: int, T: int, Smax: int) -> torch.Tensor:
    """int32 [B] cache lengths, checked on the host: each in [0, Smax - T],
    the room a T-token block's keys need (dflash_attn_prep never writes
    outside [0, Smax) and flags a sequence that would)."""
    lens_t = torch.as_tensor(lens, dtype=torch.int32).reshape(-1)
    if lens_t.numel() != B:
        raise ValueError(f"lens has {lens_t.numel()} entries for {B} sequences")
    if B and (int(lens_t.min()) < 0 or int(lens_t.max()) + T > Smax):
        raise ValueError(f"cache lengths {lens_t.tolist()} leave no room for a {T}-token block in "
                         f"{Smax} positions (need 0 <= len <= {Smax - T})")
    return lens_t


class _Plan:
    """Launch arguments of one step at one block length: the forward through
    the final norm (``fwd``), the fused LM-head accept (``lm``), the commit
    (``commit``) and the conv-window rollback from a snapshot (``conv_from``);
    each entry is (entry point, arguments without the stream)."""

    def __init__(self, T):
        self.T = T
        self.fwd: list = []
        self.lm = None
        self.commit: list = []
        self.conv_from = None


class HybridVerifyRunner:
    """One verify step (forward, greedy accept, commit) of the hybrid target
    for B sequences of up to T block tokens, with caches of Smax positions.

    Every buffer is allocated once at (B, T, Smax).  A step of any block
    length T' <= T runs on the same buffers (rows [0, B*T') of each
    activation, token slabs [0, T') of each tape) with launch arguments
    built once per T' (``forward(T')``, ``commit(T')``); the device-driven
    serving loop uses T' = T, the reference-API facade any T' (prompt
    pieces, single tokens, chunked verify)."""

    def __init__(self, cfg: HybridConfig, weights: HybridWeights, B: int, T: int, Smax: int,
                 device: torch.device, weight_layout: str = "tiled", fused_prologue: bool = True,
                 fused_norms: bool = True):
        """weight_layout: "tiled" streams weights re-laid out once as MFMA
        fragments (dflash_weight_tile_bf16, cached in the layer dicts as
        "<name>_tiled"; same sums bit for bit) wherever the row count is a
        multiple of 16 (the rest stay row-major), "rowmajor" streams the
        nn.Linear [N, K] weights as they are.  fused_prologue: each
        gated-delta layer's scan computes its own prologue
        (dflash_gdn_prologue_scan_rollback, one launch, same bits) instead of
        a prologue launch then the scan.  fused_norms (tiled weights): the
        residual adds and RMSNorms between projections run inside them
        (dflash_gemm_bf16_tiled_residual_norm adds the branch to h and stores
        h's row sums of squares, the next projection normalizes on load) instead
        of an add + RMSNorm launch per norm; the producing projections then
        split K inside a workgroup instead of across workgroups, so their
        sums (and what follows) differ from the launch form in rounding."""
        if weight_layout not in ("tiled", "rowmajor"):
            raise ValueError(f"weight_layout must be 'tiled' or 'rowmajor', got {weight_layout!r}")
        self.tiled = weight_layout == "tiled"
        self.fused_norms = bool(fused_norms) and self.tiled
        self.fused_prologue = bool(fused_prologue) and cfg.linear.linear_key_head_dim == 128
        if B < 1 or T < 1 or T > 16 or B * T > 64:
            raise ValueError("the verify step takes 1 <= T <= 16 block tokens and B*T <= 64 rows")
        if Smax <= 0 or Smax % 64:
            raise ValueError("Smax must be a positive multiple of 64")
        self.cfg, self.w, self.B, self.T, self.Smax, self.device = cfg, weights, B, T, Smax, device
        lc = cfg.linear
        M, H, I = B * T, cfg.hidden_size, cfg.intermediate_size
        bf, f32, i32 = torch.bfloat16, torch.float32, torch.int32
        z = lambda *s, dt=bf: torch.zeros(*s, dtype=dt, device=device)  # noqa: E731
        e = lambda *s, dt=bf: torch.empty(*s, dtype=dt, device=device)  # noqa: E731
        C, Hv = lc.conv_dim, lc.linear_num_value_heads
        Dk, Dv, K1 = lc.linear_key_head_dim, lc.linear_value_head_dim, lc.linear_conv_kernel_dim - 1
        Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.tokens = z(B, T, dt=i32)
        self.h = e(M, H)
        self.xn = e(M, H)
        self.r = e(M, H)
        self.mlp_act = e(M, I)
        # fused norms: the per-16-column row sums of h^2 a producing projection
        # hands the next (normed) projection
        self.row_sumsq = z(max(H // 16, 1) * M, dt=f32)
        # gated-delta layers: per-layer projection rows (the conv rollback reads
        # their qkv part after the accept), conv window, state, tape
        nl, na = cfg.n_linear, cfg.n_attention
        self.proj = [e(M, cfg.in_proj_rows) for _ in range(nl)]
        self.conv_all = z(nl, B, K1, C)
        self.conv = list(self.conv_all.unbind(0))
        self.conv_snap = None  # [nl, B, K1, C], made by snapshot_conv()
        self.state = [z(B, Hv, Dv, Dk, dt=f32) for _ in range(nl)]
        self.tape = [z(T, B, Hv, Dv, Dk, dt=f32) for _ in range(nl)]
        self.act = e(B, T, C)
        self.g = e(B, T, Hv, dt=f32)
        self.beta = e(B, T, Hv, dt=f32)
        self.conv_scratch = e(B, K1, C)
        self.scan_out = e(B, T, Hv, Dv)
        self.gnorm = e(B, T, Hv, Dv)
        # attention layers: KV caches (zero-filled: positions past the live
        # length are read with zero weight and must stay finite)
        self.aproj = e(M, cfg.attn_proj_rows)
        self.k_cache = [z(B, Hkv, Smax, D) for _ in range(na)]
        self.vt_cache = [z(B, Hkv, D, Smax) for _ in range(na)]
        self.q = e(B, T, Hq, D)
        self.attn_out = e(M, Hq * D)
        lib = _lib.load()
        self.attn_ws = e(int(lib.dflash_attn_verify_workspace_bytes(B, Hq, Hkv, Smax)), dt=torch.uint8)
        # accept / commit
        self.lens = z(B, dt=i32)
        self.keep = z(B, dt=i32)  # 0: the first step starts from `state`
        self.overflow = z(B, dt=i32)  # set by attn_prep for a block outside the cache
        self.posterior = e(B, T, dt=i32)
        self.matched = z(B, dt=i32)
        self.bonus = e(B, dt=i32)
        V = cfg.vocab_size
        self.lm_ws = e(max(int(lib.dflash_lm_head_accept_workspace_bytes(B, T, V)), 8), dt=torch.uint8)
        # the tiled GEMMs' tail split: counters zeroed once here, left zeroed by every call
        self.gemm_ws = z(int(lib.dflash_gemm_tail_workspace_bytes()), dt=torch.uint8)
        self.capture_layers: tuple[int, ...] = ()
        self.captured = None  # [B*T, len(capture_layers) * H] after set_capture
        self._plans: dict[int, _Plan] = {}
        self._prepare_weights()
        self.graph = None

    # ------------------------------------------------------------------ setup
    # (requested splits, weight rows per wave, waves sharing a row group) per
    # projection, from a sweep of cold-weight timings at M = 16 on MI355X:
    # bf16 output where the next kernel needs it as bf16, fp32 split-K
    # partials where the next add + RMSNorm sums them.
    GEMM_PLAN = {"w_in": (1, 32, 4), "w_out": (8, 16, 4), "w_qkv": (1, 32, 4),
                 "w_o": (8, 32, 4), "w_gu": (1, 32, 4), "w_down": (8, 32, 4)}
    # the same for fragment-tiled weights (rows_per_wave 64 exists only
    # there), timed inside the whole graph-captured c4 step (which also counts
    # the add + RMSNorm reading fewer partials): down in 6 splits (24 of its
    # 144 k-steps each, 6 per wave) beat 8 by ~30 us per step; with
    # nontemporal weight loads, out_proj in 6 splits and down at 64 rows per
    # wave save another ~19 us
    TILED_PLAN = {"w_in": (1, 64, 4), "w_out": (6, 32, 4), "w_qkv": (1, 32, 4),
                  "w_o": (8, 16, 4), "w_gu": (1, 32, 4), "w_down": (6, 64, 4)}

    def _dims(self):
        cfg, lc, H, I = self.cfg, self.cfg.linear, self.cfg.hidden_size, self.cfg.intermediate_size
        return {"w_in": (cfg.in_proj_rows, H), "w_out": (H, lc.value_dim),
                "w_qkv": (cfg.attn_proj_rows, H),
                "w_o": (H, cfg.num_attention_heads * cfg.head_dim),
                "w_gu": (2 * I, H), "w_down": (H, I)}

    def _prepare_weights(self):
        """Split counts, the split-K partial buffer (fp32 [splits, M, N],
        shared by the consumers in order) and the derived weight copies (made
        once per weight set, cached in the layer dicts): gate|up rows paired
        for the fused SwiGLU GEMM, fragment-tiled copies, the tiled LM head."""
        cfg, M, H, I = self.cfg, self.B * self.T, self.cfg.hidden_size, self.cfg.intermediate_size
        dims = self._dims()
        lib = _lib.load()
        self.plan = self.TILED_PLAN if self.tiled else self.GEMM_PLAN
        self.splits = {k: int(lib.dflash_gemm_splits(dims[k][1], p[0])) if p[0] > 1 else 0
                       for k, p in self.plan.items()}
        part_elems = max([self.splits[k] * M * dims[k][0] for k in dims] + [1])
        self.part = torch.empty(part_elems, dtype=torch.float32, device=self.device)
        stream = _lib.stream_handle(self.device)

        def tile(lw, key):
            tkey = key + "_tiled"
            if tkey not in lw:
                w = lw[key]
                n, k = w.shape
                t = torch.empty(int(lib.dflash_weight_tile_bytes(n, k)) // 2, dtype=torch.bfloat16,
                                device=self.device)
                _lib.call("dflash_weight_tile_bf16", w.data_ptr(), w.stride(0), t.data_ptr(), n, k,
                          stream)
                lw[tkey] = t

        for i, lw in enumerate(self.w.layers):
            if "w_gu_pairs" not in lw:
                # [gate; up] rows regrouped into 32-row blocks (16 gate rows,
                # then the 16 up rows of the same columns)
                lw["w_gu_pairs"] = lw["w_gu"].view(2, I // 16, 16, H).transpose(0, 1) \
                    .reshape(2 * I, H).contiguous()
            if self.tiled:
                names = ["w_gu_pairs", "w_down"] + (["w_in", "w_out"] if cfg.is_linear(i)
                                                    else ["w_qkv", "w_o"])
                for name in names:
                    n = lw[name].shape[0]
                    if n % 16 == 0:  # the fragment layout needs whole 16-row tiles
                        tile(lw, name)
        if self.fused_norms and not (all(self.plan[n][2] == 4 for n in ("w_in", "w_qkv", "w_gu"))
                                     and H % 16 == 0 and H <= 16384):
            self.fused_norms = False  # the normed projections stream with k_waves == 4
        if self.tiled and cfg.vocab_size % 16 == 0 and self.w.lm_head_tiled is None:
            from .runtime import tile_weight

            self.w.lm_head_tiled = tile_weight(self.w.lm_head)
        torch.cuda.synchronize(self.device)

    def set_capture(self, layer_ids) -> None:
        """Store the residual stream after each layer in layer_ids (in layer
        order) to self.captured [B*T, n * H] on every forward: the target
        hidden states of forward_dflash (custom_qwen35_model.py:984-991)."""
        ids = tuple(sorted({int(i) for i in layer_ids}))
        if ids and not 0 <= ids[0] <= ids[-1] < self.cfg.num_hidden_layers:
            raise ValueError(f"layer_ids {list(layer_ids)} outside [0, {self.cfg.num_hidden_layers})")
        if ids == self.capture_layers:
            return
        self.capture_layers = ids
        H = self.cfg.hidden_size
        self.captured = (torch.empty(self.B * self.T, len(ids) * H, dtype=torch.bfloat16,
                                     device=self.device) if ids else None)
        self._plans.clear()
        self.graph = None

    def _plan(self, T: int) -> _Plan:
        p = self._plans.get(T)
        if p is None:
            if not 1 <= T <= self.T:
                raise ValueError(f"block length {T} outside [1, {self.T}]")
            p = self._plans[T] = self._build_plan(T)
        return p

    def _gemm_op(self, lw, name, x, out_ptr, out_stride, M):
        n, k = self._dims()[name]
        ns, rpw, kw = self.plan[name]
        if self.tiled and name + "_tiled" in lw:
            return ("dflash_gemm_bf16_tiled",
                    (x.data_ptr(), x.stride(0), lw[name + "_tiled"].data_ptr(), out_ptr, out_stride,
                     M, n, k, ns, rpw, kw) + self._gemm_ws(kw))
        w = lw[name]
        # row-major kernel widths; the split count stays the one the consumers
        # were set up for
        rpw, kw = self.GEMM_PLAN[name][1], self.GEMM_PLAN[name][2]
        return ("dflash_gemm_bf16", (x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), out_ptr,
                                     out_stride, M, n, k, ns, rpw, kw))

    def _fusable(self, lw, *names) -> bool:
        """The fused-norm forms apply: every named projection of this layer
        has its tiled copy."""
        return self.fused_norms and all(n + "_tiled" in lw for n in names)

    def _residual_norm_op(self, lw, name, x, M, capture):
        """Projection `name` with h += its output and the row sums of h^2 (per
        16 columns) for the next (normed) projection."""
        n, k = self._dims()[name]
        cap, cap_stride = capture if capture is not None else (None, 0)
        return ("dflash_gemm_bf16_tiled_residual_norm",
                (x.data_ptr(), x.stride(0), lw[name + "_tiled"].data_ptr(), M, n, k,
                 self.h.data_ptr(), self.h.data_ptr(), cap, cap_stride, self.row_sumsq.data_ptr()))

    def _gemm_ws(self, k_waves):
        """The tail-split workspace of the k_waves 4 tiled GEMMs (none for 1)."""
        if k_waves != 4:
            return (None, 0)
        return (self.gemm_ws.data_ptr(), self.gemm_ws.numel())

    def _norm_input(self, w_norm):
        """Arguments of a normed projection's input: RMSNorm(h) with weight
        w_norm, from the producing call's row sums."""
        H = self.cfg.hidden_size
        return (self.h.data_ptr(), self.h.stride(0), w_norm.data_ptr(), self.row_sumsq.data_ptr(),
                H // 16, float(self.cfg.rms_norm_eps), None)

    def _residual_op(self, name, w_norm, M, capture):
        """h += the branch projection `name` just produced; xn = norm(h);
        capture = (pointer, row stride) also receives h."""
        H, eps = self.cfg.hidden_size, float(self.cfg.rms_norm_eps)
        h, xn, ns = self.h.data_ptr(), self.xn.data_ptr(), self.splits[name]
        if capture is not None:
            rp = self.part.data_ptr() if ns else None
            r = None if ns else self.r.data_ptr()
            return ("dflash_add_rmsnorm_capture",
                    (h, r, rp, ns, w_norm.data_ptr(), h, capture[0], capture[1], xn, M, H, eps))
        if ns:
            return ("dflash_add_rmsnorm_splitk",
                    (h, self.part.data_ptr(), ns, w_norm.data_ptr(), h, xn, M, H, eps))
        return ("dflash_add_rmsnorm", (h, self.r.data_ptr(), w_norm.data_ptr(), h, xn, M, H, eps))

    def _build_plan(self, T: int) -> _Plan:
        cfg, lc, B = self.cfg, self.cfg.linear, self.B
        M, H, I = B * T, cfg.hidden_size, cfg.intermediate_size
        C, Hk, Hv = lc.conv_dim, lc.linear_num_key_heads, lc.linear_num_value_heads
        Dk, Dv, K = lc.linear_key_head_dim, lc.linear_value_head_dim, lc.linear_conv_kernel_dim
        Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        rows, arows = cfg.in_proj_rows, cfg.attn_proj_rows
        eps = float(cfg.rms_norm_eps)
        pl = _Plan(T)
        pp = self.part.data_ptr()
        # host arrays handed to the library by pointer live as long as the plan
        pl.keep_alive = []

        def dst(name, bf16_out):
            return (pp, 0) if self.splits[name] else (bf16_out.data_ptr(), bf16_out.stride(0))

        cap_index = {layer: j for j, layer in enumerate(self.capture_layers)}
        cap_stride = len(self.capture_layers) * H

        def capture_of(layer):
            j = cap_index.get(layer)
            return None if j is None else (self.captured.data_ptr() + 2 * j * H, cap_stride)

        ab_strides = (ctypes.c_int64 * 4)(T * rows, rows, T * rows, rows)
        z_strides = (ctypes.c_int64 * 3)(T * rows, rows, Dv)
        scan_strides = (ctypes.c_int64 * 13)(
            T * C, C, Dk, T * C, C, Dk, T * C, C, Dv, T * Hv, Hv, T * Hv, Hv)
        pl.keep_alive += [ab_strides, z_strides, scan_strides]
        act = self.act.data_ptr()
        fwd = pl.fwd
        fwd.append(("dflash_embed_rmsnorm",
                    (self.w.embed.data_ptr(), self.tokens.data_ptr(), cfg.vocab_size,
                     self.w.layers[0]["ln_in"].data_ptr(), self.h.data_ptr(), self.xn.data_ptr(),
                     M, H, eps)))
        L = cfg.num_hidden_layers
        gi = ai = 0
        for i in range(L):
            lw = self.w.layers[i]
            if i > 0:
                fwd.append(self._residual_op("w_down", lw["ln_in"], M, capture_of(i - 1)))
            # the post-attention norm folds when this layer's output projection
            # and its gate|up GEMM both have tiled copies
            post = self._fusable(lw, "w_out" if cfg.is_linear(i) else "w_o", "w_gu_pairs")
            if cfg.is_linear(i):
                gw = lw["gdn"]
                base = self.proj[gi].data_ptr()
                fwd.append(self._gemm_op(lw, "w_in", self.xn, *dst("w_in", self.proj[gi]), M))
                conv = self.conv[gi].data_ptr()
                a_ptr, b_ptr = base + 2 * (C + Hv * Dv + Hv), base + 2 * (C + Hv * Dv)
                state, tape = self.state[gi].data_ptr(), self.tape[gi].data_ptr()
                keep = self.keep.data_ptr()
                out = self.scan_out.data_ptr()
                if self.fused_prologue:
                    fwd.append(("dflash_gdn_prologue_scan_rollback",
                                (base, T * rows, rows, conv, gw.conv_weight.data_ptr(), a_ptr, b_ptr,
                                 ab_strides, gw.A_log.data_ptr(), gw.dt_bias.data_ptr(), state, tape,
                                 keep, self.T, B, out, None, tape, B, T, K, Hk, Hv, Dk, Dv,
                                 QK_NORM_EPS)))
                else:
                    fwd.append(("dflash_gdn_prologue",
                                (base, T * rows, rows, conv, gw.conv_weight.data_ptr(), a_ptr, b_ptr,
                                 ab_strides, gw.A_log.data_ptr(), gw.dt_bias.data_ptr(), act,
                                 self.g.data_ptr(), self.beta.data_ptr(), self.conv_scratch.data_ptr(),
                                 B, T, K, Hk, Hv, Dk, Dv, QK_NORM_EPS)))
                    fwd.append(("dflash_gdn_verify_scan_rollback",
                                (act, act + 2 * Hk * Dk, act + 4 * Hk * Dk, self.g.data_ptr(),
                                 self.beta.data_ptr(), state, tape, keep, self.T, B, out, None, tape,
                                 B, T, Hk, Hv, Dk, Dv, scan_strides)))
                fwd.append(("dflash_gdn_gated_rmsnorm",
                            (out, base + 2 * C, z_strides, gw.norm_weight.data_ptr(),
                             self.gnorm.data_ptr(), B, T, Hv, Dv, eps)))
                if post:
                    fwd.append(self._residual_norm_op(lw, "w_out", self.gnorm.view(-1, Hv * Dv), M,
                                                      None))
                else:
                    fwd.append(self._gemm_op(lw, "w_out", self.gnorm.view(-1, Hv * Dv),
                                             *dst("w_out", self.r), M))
                    fwd.append(self._residual_op("w_out", lw["ln_post"], M, None))
                gi += 1
            else:
                fwd.append(self._gemm_op(lw, "w_qkv", self.xn, *dst("w_qkv", self.aproj), M))
                if self.splits["w_qkv"]:
                    fwd.append(("dflash_splitk_reduce", (pp, self.splits["w_qkv"], M, arows,
                                                         self.aproj.data_ptr(), arows)))
                fwd.append(("dflash_attn_prep",
                            (self.aproj.data_ptr(), arows, lw["q_norm"].data_ptr(),
                             lw["k_norm"].data_ptr(), self.lens.data_ptr(),
                             self.k_cache[ai].data_ptr(), self.vt_cache[ai].data_ptr(),
                             self.q.data_ptr(), self.overflow.data_ptr(), B, T, Hq, Hkv, D,
                             self.Smax, cfg.rot_dims, float(cfg.rope_theta), eps)))
                fwd.append(("dflash_attn_verify",
                            (self.q.data_ptr(), self.k_cache[ai].data_ptr(),
                             self.vt_cache[ai].data_ptr(), self.lens.data_ptr(),
                             self.aproj.data_ptr(), arows, self.attn_out.data_ptr(), B, T, Hq, Hkv,
                             D, self.Smax, self.Smax, float(D ** -0.5), self.attn_ws.data_ptr(),
                             self.attn_ws.numel())))
                if post:
                    fwd.append(self._residual_norm_op(lw, "w_o", self.attn_out, M, None))
                else:
                    fwd.append(self._gemm_op(lw, "w_o", self.attn_out, *dst("w_o", self.r), M))
                    fwd.append(self._residual_op("w_o", lw["ln_post"], M, None))
                ai += 1
            gu_key = "w_gu_pairs_tiled" if self.tiled and "w_gu_pairs_tiled" in lw else None
            if post:
                fwd.append(("dflash_gemm_bf16_swiglu_tiled_normed",
                            self._norm_input(lw["ln_post"]) + (lw[gu_key].data_ptr(),
                                                               self.mlp_act.data_ptr(), I, M, 2 * I,
                                                               H, self.plan["w_gu"][2])
                            + self._gemm_ws(self.plan["w_gu"][2])))
            elif gu_key:
                fwd.append(("dflash_gemm_bf16_swiglu_tiled",
                            (self.xn.data_ptr(), H, lw[gu_key].data_ptr(), self.mlp_act.data_ptr(),
                             I, M, 2 * I, H, self.plan["w_gu"][2]) + self._gemm_ws(self.plan["w_gu"][2])))
            else:
                fwd.append(("dflash_gemm_bf16_swiglu",
                            (self.xn.data_ptr(), H, lw["w_gu_pairs"].data_ptr(), H,
                             self.mlp_act.data_ptr(), I, M, 2 * I, H, self.plan["w_gu"][2])))
            # The next layer's input norm stays a launch: the down projection
            # (K = intermediate) streams faster split over workgroups than as
            # one workgroup per 16 columns, by more than the launch costs.
            fwd.append(self._gemm_op(lw, "w_down", self.mlp_act, *dst("w_down", self.r), M))
        fwd.append(self._residual_op("w_down", self.w.final_norm, M, capture_of(L - 1)))
        # LM head + greedy accept: draft = block[1:] of each sequence (row stride T)
        tail = (self.tokens.data_ptr() + 4, T, T - 1, self.posterior.data_ptr(),
                self.matched.data_ptr(), self.bonus.data_ptr(), B, T, self.lm_ws.data_ptr(),
                self.lm_ws.numel())
        if self.w.lm_head_tiled is not None and self.tiled:
            pl.lm = ("dflash_lm_head_greedy_accept_tiled",
                     (self.xn.data_ptr(), H, self.w.lm_head_tiled.data_ptr(), H, cfg.vocab_size)
                     + tail)
        else:
            pl.lm = ("dflash_lm_head_greedy_accept",
                     (self.xn.data_ptr(), H, self.w.lm_head.data_ptr(), H, H, cfg.vocab_size) + tail)
        # commit: keep = matched + 1, lens += keep, conv windows rolled to keep
        cin = _lib.ptr_array(self.conv)
        qkv = _lib.ptr_array(self.proj)
        pl.keep_alive += [cin, qkv]
        K1 = K - 1
        pl.commit = [
            ("dflash_commit_accept", (self.matched.data_ptr(), self.keep.data_ptr(),
                                      self.lens.data_ptr(), B, T)),
            ("dflash_conv_rollback", (cin, qkv, cin, self.keep.data_ptr(), cfg.n_linear, B, T, K1, C,
                                      T * rows, rows, 2)),
        ]
        if self.conv_snap is not None:
            snap = _lib.ptr_array(list(self.conv_snap.unbind(0)))
            pl.keep_alive.append(snap)
            pl.conv_from = ("dflash_conv_rollback", (snap, qkv, cin, self.keep.data_ptr(),
                                                     cfg.n_linear, B, T, K1, C, T * rows, rows, 2))
        return pl

    # ------------------------------------------------------------ cache I/O
    def set_state(self, lens, conv=None, rec=None, k=None, v=None):
        """Load cache contents: lens [B] (live KV length), per gated-delta layer
        conv windows [B,K-1,C] and states [B,Hv,Dv,Dk], per attention layer
        keys / values [B,Hkv,S<=Smax,D] (positions >= S are zeroed).  Clears the
        pending accept (the next step starts from `rec`) and the overflow
        flags.  Raises unless 0 <= lens[b] and lens[b] + T <= Smax, the room
        the next block's keys need."""
        self.lens.copy_(check_cache_lengths(lens, self.B, self.T, self.Smax))
        self.keep.zero_()
        self.overflow.zero_()
        for dst, src in ((self.conv, conv), (self.state, rec)):
            if src is not None:
                for d_, s_ in zip(dst, src):
                    d_.copy_(s_)
        if k is not None:
            for kc, vc, kk, vv in zip(self.k_cache, self.vt_cache, k, v):
                S = kk.shape[2]
                if S > self.Smax:
                    raise ValueError(f"{S} cached positions exceed Smax = {self.Smax}")
                kc.zero_()
                vc.zero_()
                kc[:, :, :S].copy_(kk)
                vc[:, :, :, :S].copy_(vv.transpose(2, 3))

    def check_overflow(self) -> None:
        """Raise if any step since the last set_state / clear wrote a block
        outside its cache (dflash_attn_prep's overflow flags; one sync)."""
        bad = self.overflow.nonzero().flatten().tolist()
        if bad:
            raise RuntimeError(f"sequences {bad} ran a block past their {self.Smax}-position KV "
                               "cache; their outputs are invalid")

    def snapshot_conv(self) -> None:
        """Copy every conv window to conv_snap (the initial windows a later
        rollback_to() restarts from)."""
        if self.conv_snap is None:
            self.conv_snap = torch.empty_like(self.conv_all)
            self._plans.clear()
            self.graph = None
        self.conv_snap.copy_(self.conv_all)

    # ------------------------------------------------------------------- step
    def _run(self, ops) -> None:
        stream = _lib.stream_handle(self.device)
        call = _lib.call
        for fn, args in ops:
            call(fn, *args, stream)

    def forward(self, T: int | None = None, lm_head: bool = True) -> None:
        """Embed tokens [B, T'] (packed at the start of self.tokens), run the
        layers and the final norm (xn = the normed hidden states, captured
        layers to self.captured) and, with lm_head, the fused LM-head greedy
        accept into posterior / matched / bonus (draft = block[1:]).  The
        recurrent states are rolled back on load to the previous step's keep
        counts."""
        p = self._plan(self.T if T is None else int(T))
        self._run(p.fwd)
        if lm_head:
            self._run([p.lm])

    def forward_accept(self) -> None:
        """forward() of a full T-token block with the fused LM-head accept."""
        self.forward(self.T, lm_head=True)

    def commit(self, T: int | None = None) -> None:
        """keep = matched + 1, lens += keep, and every conv window rolled to
        keep tokens (the recurrent states follow on the next step's load)."""
        self._run(self._plan(self.T if T is None else int(T)).commit)

    def accept_all(self, T: int) -> None:
        """Keep every token of the last T-token block: keep = T (the states
        follow tape[T-1] on the next load) and the conv windows advanced by
        the block's qkv rows, in place.  The KV lengths stay with the caller."""
        p = self._plan(int(T))
        self.keep.fill_(int(T))
        self._run(p.commit[1:])

    def rollback_to(self, T: int) -> None:
        """Conv windows rebuilt from conv_snap and the block's qkv rows at the
        device-side keep counts (the state follows on the next load)."""
        p = self._plan(int(T))
        if p.conv_from is None:
            raise RuntimeError("rollback_to needs snapshot_conv() before the forward")
        self._run([p.conv_from])

    def step(self):
        self.forward_accept()
        self.commit()

    # ------------------------------------------------------------- HIP graph
    def capture_step(self):
        """Capture one step (forward, accept, commit) as a HIP graph.  The
        capture itself does not execute the step."""
        self._plan(self.T)  # build outside the capture
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=s):
            self.step()
        torch.cuda.synchronize(self.device)
        return self.graph

    def replay(self):
        self.graph.replay()

    # --------------------------------------------------------------- readout
    def committed_states(self):
        """Per gated-delta layer, the recurrent state after the last commit:
        tape[keep-1] (or the loaded state when nothing was committed yet)."""
        keep = self.keep.cpu().tolist()
        out = []
        for st, tp in zip(self.state, self.tape):
            out.append(torch.stack([tp[k - 1, b] if k >= 1 else st[b] for b, k in enumerate(keep)]))
        return out
