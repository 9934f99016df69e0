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
  the gate|up projection), or as plain bf16
  ``torch.mm`` on hipBLASLt (``gemm="hipblaslt"``);
* everything else on this package's gfx950 kernels through the C ABI:
  residual add + RMSNorm, the gated-delta prologue, the scan with the previous
  step's rollback fused into its state load (per-token tape), the gated
  RMSNorm, q/k norm + rotary + KV append, split-K verify attention + gate,
  SwiGLU, the fused LM-head greedy accept, and the commit (keep counts, KV
  lengths, conv windows).

Cache lengths and accept counts stay in device memory and no step reads
anything back to the host, so one step can be captured as a HIP graph and
replayed (``capture_step`` / ``replay``).

Random-init weights (bf16 ~ N(0, std) for every projection, unit norms, the
reference's gated-delta parameter inits) and synthetic caches stand in for a
checkpoint; there is no network here.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from . import _lib
from .gdn_layer import GatedDeltaConfig, GatedDeltaWeights


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


class HybridVerifyRunner:
    """One verify step (forward, greedy accept, commit) of the hybrid target
    for B sequences of T block tokens, with caches of Smax positions."""

    def __init__(self, cfg: HybridConfig, weights: HybridWeights, B: int, T: int, Smax: int,
                 device: torch.device, gemm: str = "dflash", weight_layout: str = "tiled",
                 fused_prologue: bool = True):
        """gemm: "dflash" runs every projection on this package's verify-sized
        GEMM (split-K partials summed by the consumer); "hipblaslt" runs them
        as torch.mm (for comparison).  weight_layout (dflash GEMMs): "tiled"
        streams weights re-laid out once as MFMA fragments
        (dflash_weight_tile_bf16, cached in the layer dicts as "<name>_tiled";
        same sums bit for bit) wherever the row count is a multiple of 16 (the
        rest stay row-major), "rowmajor" streams the nn.Linear [N, K] weights
        as they are.  fused_prologue (dflash GEMMs): each gated-delta layer's
        scan computes its own prologue (dflash_gdn_prologue_scan_rollback, one
        launch, same bits) instead of a prologue launch then the scan."""
        if gemm not in ("dflash", "hipblaslt"):
            raise ValueError(f"gemm must be 'dflash' or 'hipblaslt', got {gemm!r}")
        if weight_layout not in ("tiled", "rowmajor"):
            raise ValueError(f"weight_layout must be 'tiled' or 'rowmajor', got {weight_layout!r}")
        self.gemm = gemm
        self.tiled = weight_layout == "tiled"
        self.fused_prologue = bool(fused_prologue) and cfg.linear.linear_key_head_dim == 128
        if T > 16 or B * T > 64:
            raise ValueError("the verify step takes T <= 16 block tokens and B*T <= 64 rows")
        if Smax % 64:
            raise ValueError("Smax must be a multiple of 64")
        self.cfg, self.w, self.B, self.T, self.Smax, self.device = cfg, weights, B, T, Smax, device
        lc = cfg.linear
        M, H, I = B * T, cfg.hidden_size, cfg.intermediate_size
        bf, f32, i32 = torch.bfloat16, torch.float32, torch.int32
        z = lambda *s, dt=bf: torch.zeros(*s, dtype=dt, device=device)  # noqa: E731
        e = lambda *s, dt=bf: torch.empty(*s, dtype=dt, device=device)  # noqa: E731
        C, Hk, Hv = lc.conv_dim, lc.linear_num_key_heads, lc.linear_num_value_heads
        Dk, Dv, K1 = lc.linear_key_head_dim, lc.linear_value_head_dim, lc.linear_conv_kernel_dim - 1
        Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.tokens = z(B, T, dt=i32)
        self.h = e(M, H)
        self.xn = e(M, H)
        self.r = e(M, H)
        self.gu = e(M, 2 * I)
        self.mlp_act = e(M, I)
        # gated-delta layers: per-layer projection rows (the conv rollback reads
        # their qkv part after the accept), conv window, state, tape
        nl, na = cfg.n_linear, cfg.n_attention
        self.proj = [e(M, cfg.in_proj_rows) for _ in range(nl)]
        self.conv = [z(B, K1, C) for _ in range(nl)]
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
        self.posterior = e(B, T, dt=i32)
        self.matched = z(B, dt=i32)
        self.bonus = e(B, dt=i32)
        V = cfg.vocab_size
        self.lm_ws = e(max(int(lib.dflash_lm_head_accept_workspace_bytes(B, T, V)), 8), dt=torch.uint8)
        self._build_gemms()
        self._build_args()
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

    def _build_gemms(self):
        """Argument tuples of every projection GEMM, and the split-K partial
        buffer (fp32 [splits, M, N]) shared by the consumers in order."""
        cfg, B, T = self.cfg, self.B, self.T
        M, H, I = B * T, cfg.hidden_size, cfg.intermediate_size
        lc = cfg.linear
        dims = {"w_in": (cfg.in_proj_rows, H), "w_out": (H, lc.value_dim),
                "w_qkv": (cfg.attn_proj_rows, H),
                "w_o": (H, cfg.num_attention_heads * cfg.head_dim),
                "w_gu": (2 * I, H), "w_down": (H, I)}
        lib = _lib.load()
        plan_of = self.TILED_PLAN if self.tiled else self.GEMM_PLAN
        self.plan = plan_of
        self.splits = {k: int(lib.dflash_gemm_splits(dims[k][1], plan[0])) if plan[0] > 1 else 0
                       for k, plan in plan_of.items()}
        part_elems = max([self.splits[k] * M * dims[k][0] for k in dims] + [1])
        self.part = torch.empty(part_elems, dtype=torch.float32, device=self.device)
        pp = self.part.data_ptr()

        stream = _lib.stream_handle(self.device)

        def tiled(lw, key, w):
            """The fragment-tiled copy of weight w, made once per weight set."""
            tkey = key + "_tiled"
            if tkey not in lw:
                n, k = w.shape
                t = torch.empty(int(lib.dflash_weight_tile_bytes(n, k)) // 2, dtype=torch.bfloat16,
                                device=self.device)
                _lib.call("dflash_weight_tile_bf16", w.data_ptr(), w.stride(0), t.data_ptr(), n, k,
                          stream)
                lw[tkey] = t
            return lw[tkey]

        def args(lw, x, name, out_ptr, out_stride):
            """(entry point, arguments) of projection `name` of layer dict lw."""
            n, k = dims[name]
            ns, rpw, kw = plan_of[name]
            if self.tiled and n % 16 == 0:  # the fragment layout needs whole 16-row tiles
                return ("dflash_gemm_bf16_tiled",
                        (x.data_ptr(), x.stride(0), tiled(lw, name, lw[name]).data_ptr(), out_ptr,
                         out_stride, M, n, k, ns, rpw, kw))
            w = lw[name]
            # row-major kernel widths; the split count stays the one the
            # consumers were set up for
            rpw, kw = self.GEMM_PLAN[name][1], self.GEMM_PLAN[name][2]
            return ("dflash_gemm_bf16", (x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                                         out_ptr, out_stride, M, n, k, ns, rpw, kw))

        def gate_up_pairs(lw):
            """w_gu [gate; up] rows regrouped into 32-row blocks (16 gate rows,
            then the 16 up rows of the same columns) for the fused-SwiGLU GEMM;
            made once per weight set."""
            if "w_gu_pairs" not in lw:
                w = lw["w_gu"]
                lw["w_gu_pairs"] = w.view(2, I // 16, 16, H).transpose(0, 1).reshape(2 * I, H) \
                    .contiguous()
            return lw["w_gu_pairs"]

        def dst(name, bf16_out):
            return (pp, 0) if self.splits[name] else (bf16_out.data_ptr(), bf16_out.stride(0))

        self._gemm_args = []
        gi = 0
        for i in range(cfg.num_hidden_layers):
            lw = self.w.layers[i]
            wp = gate_up_pairs(lw)
            if self.tiled:
                gu = ("dflash_gemm_bf16_swiglu_tiled",
                      (self.xn.data_ptr(), H, tiled(lw, "w_gu_pairs", wp).data_ptr(),
                       self.mlp_act.data_ptr(), I, M, 2 * I, H, plan_of["w_gu"][2]))
            else:
                gu = ("dflash_gemm_bf16_swiglu",
                      (self.xn.data_ptr(), H, wp.data_ptr(), H, self.mlp_act.data_ptr(), I, M, 2 * I,
                       H, plan_of["w_gu"][2]))
            a = {"gu": gu, "down": args(lw, self.mlp_act, "w_down", *dst("w_down", self.r))}
            if cfg.is_linear(i):
                a["in"] = args(lw, self.xn, "w_in", *dst("w_in", self.proj[gi]))
                a["out"] = args(lw, self.gnorm.view(M, -1), "w_out", *dst("w_out", self.r))
                gi += 1
            else:
                a["qkv"] = args(lw, self.xn, "w_qkv", *dst("w_qkv", self.aproj))
                a["o"] = args(lw, self.attn_out, "w_o", *dst("w_o", self.r))
            self._gemm_args.append(a)
        torch.cuda.synchronize(self.device)

    def _residual(self, name, w_norm, stream):
        """h += the branch just produced by projection `name`; xn = norm(h)."""
        cfg = self.cfg
        M, H, eps = self.B * self.T, cfg.hidden_size, float(cfg.rms_norm_eps)
        h, xn = self.h.data_ptr(), self.xn.data_ptr()
        if self.splits[name]:
            _lib.call("dflash_add_rmsnorm_splitk", h, self.part.data_ptr(), self.splits[name],
                      w_norm.data_ptr(), h, xn, M, H, eps, stream)
        else:
            _lib.call("dflash_add_rmsnorm", h, self.r.data_ptr(), w_norm.data_ptr(), h, xn, M, H,
                      eps, stream)

    def _build_args(self):
        cfg, lc, B, T = self.cfg, self.cfg.linear, self.B, self.T
        C, Hk, Hv = lc.conv_dim, lc.linear_num_key_heads, lc.linear_num_value_heads
        Dk, Dv, K = lc.linear_key_head_dim, lc.linear_value_head_dim, lc.linear_conv_kernel_dim
        rows = cfg.in_proj_rows
        eps = float(cfg.rms_norm_eps)
        self._ab_strides = (ctypes.c_int64 * 4)(T * rows, rows, T * rows, rows)
        self._z_strides = (ctypes.c_int64 * 3)(T * rows, rows, Dv)
        self._scan_strides = (ctypes.c_int64 * 13)(
            T * C, C, Dk, T * C, C, Dk, T * C, C, Dv, T * Hv, Hv, T * Hv, Hv)
        self._gdn_args = []
        gi = 0
        for i in range(cfg.num_hidden_layers):
            if not cfg.is_linear(i):
                continue
            gw = self.w.layers[i]["gdn"]
            p = self.proj[gi]
            base = p.data_ptr()
            act = self.act.data_ptr()
            prologue = (base, T * rows, rows, self.conv[gi].data_ptr(), gw.conv_weight.data_ptr(),
                        base + 2 * (C + Hv * Dv + Hv), base + 2 * (C + Hv * Dv), self._ab_strides,
                        gw.A_log.data_ptr(), gw.dt_bias.data_ptr(), act, self.g.data_ptr(),
                        self.beta.data_ptr(), self.conv_scratch.data_ptr(), B, T, K, Hk, Hv, Dk, Dv,
                        eps)
            scan = (act, act + 2 * Hk * Dk, act + 4 * Hk * Dk, self.g.data_ptr(), self.beta.data_ptr(),
                    self.state[gi].data_ptr(), self.tape[gi].data_ptr(), self.keep.data_ptr(), T, B,
                    self.scan_out.data_ptr(), None, self.tape[gi].data_ptr(), B, T, Hk, Hv, Dk, Dv,
                    self._scan_strides)
            gnorm = (self.scan_out.data_ptr(), base + 2 * C, self._z_strides,
                     gw.norm_weight.data_ptr(), self.gnorm.data_ptr(), B, T, Hv, Dv, eps)
            fused = prologue[:10] + scan[5:15] + (K, Hk, Hv, Dk, Dv, eps)
            self._gdn_args.append((prologue, scan, gnorm, fused))
            gi += 1
        self._conv_ptrs = (_lib.ptr_array(self.conv), _lib.ptr_array(self.proj),
                           _lib.ptr_array(self.conv))
        Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        arows = cfg.attn_proj_rows
        self._attn_args = []
        ai = 0
        for i in range(cfg.num_hidden_layers):
            if cfg.is_linear(i):
                continue
            lw = self.w.layers[i]
            prep = (self.aproj.data_ptr(), arows, lw["q_norm"].data_ptr(), lw["k_norm"].data_ptr(),
                    self.lens.data_ptr(), self.k_cache[ai].data_ptr(), self.vt_cache[ai].data_ptr(),
                    self.q.data_ptr(), B, T, Hq, Hkv, D, self.Smax, cfg.rot_dims,
                    float(cfg.rope_theta), eps)
            attn = (self.q.data_ptr(), self.k_cache[ai].data_ptr(), self.vt_cache[ai].data_ptr(),
                    self.lens.data_ptr(), self.aproj.data_ptr(), arows, self.attn_out.data_ptr(), B, T,
                    Hq, Hkv, D, self.Smax, self.Smax, float(D ** -0.5), self.attn_ws.data_ptr(),
                    self.attn_ws.numel())
            self._attn_args.append((prep, attn))
            ai += 1
        # draft = block[1:] of each sequence (row stride T)
        tail = (self.tokens.data_ptr() + 4, T, T - 1, self.posterior.data_ptr(),
                self.matched.data_ptr(), self.bonus.data_ptr(), B, T, self.lm_ws.data_ptr(),
                self.lm_ws.numel())
        if self.tiled and self.gemm == "dflash" and cfg.vocab_size % 16 == 0:
            if self.w.lm_head_tiled is None:
                from .runtime import tile_weight

                self.w.lm_head_tiled = tile_weight(self.w.lm_head)
            self._lm_fn = "dflash_lm_head_greedy_accept_tiled"
            self._lm_args = (self.xn.data_ptr(), cfg.hidden_size, self.w.lm_head_tiled.data_ptr(),
                             cfg.hidden_size, cfg.vocab_size) + tail
        else:
            self._lm_fn = "dflash_lm_head_greedy_accept"
            self._lm_args = (self.xn.data_ptr(), cfg.hidden_size, self.w.lm_head.data_ptr(),
                             cfg.hidden_size, cfg.hidden_size, cfg.vocab_size) + tail

    def set_state(self, lens, conv=None, rec=None, k=None, v=None):
        """Load cache contents: lens [B] (live KV length), per gated-delta layer
        conv windows [B,K-1,C] and states [B,Hv,Dv,Dk], per attention layer
        keys / values [B,Hkv,S<=Smax,D] (positions >= S are zeroed).  Clears the
        pending accept (the next step starts from `rec`)."""
        self.lens.copy_(torch.as_tensor(lens, dtype=torch.int32))
        self.keep.zero_()
        for dst, src in ((self.conv, conv), (self.state, rec)):
            if src is not None:
                for d_, s_ in zip(dst, src):
                    d_.copy_(s_)
        if k is not None:
            for kc, vc, kk, vv in zip(self.k_cache, self.vt_cache, k, v):
                S = kk.shape[2]
                kc.zero_()
                vc.zero_()
                kc[:, :, :S].copy_(kk)
                vc[:, :, :, :S].copy_(vv.transpose(2, 3))

    # ------------------------------------------------------------------- step
    def _mm(self, x, w, out):
        torch.mm(x, w.t(), out=out)

    def forward_accept(self):
        """Embed self.tokens, run the 32 layers, the final norm and the fused
        LM-head greedy accept into posterior / matched / bonus.  The recurrent
        states are rolled back on load to the previous step's keep counts."""
        if self.gemm == "hipblaslt":
            return self._forward_accept_hipblaslt()
        cfg, B, T = self.cfg, self.B, self.T
        stream = _lib.stream_handle(self.device)
        call = _lib.call
        M, H, I = B * T, cfg.hidden_size, cfg.intermediate_size
        eps = float(cfg.rms_norm_eps)
        call("dflash_embed_rmsnorm", self.w.embed.data_ptr(), self.tokens.data_ptr(),
             cfg.vocab_size, self.w.layers[0]["ln_in"].data_ptr(), self.h.data_ptr(),
             self.xn.data_ptr(), M, H, eps, stream)
        gi = ai = 0
        for i in range(cfg.num_hidden_layers):
            lw = self.w.layers[i]
            ga = self._gemm_args[i]
            if i > 0:
                self._residual("w_down", lw["ln_in"], stream)
            if cfg.is_linear(i):
                prologue, scan, gnorm, fused = self._gdn_args[gi]
                call(ga["in"][0], *ga["in"][1], stream)
                if self.fused_prologue:
                    call("dflash_gdn_prologue_scan_rollback", *fused, stream)
                else:
                    call("dflash_gdn_prologue", *prologue, stream)
                    call("dflash_gdn_verify_scan_rollback", *scan, stream)
                call("dflash_gdn_gated_rmsnorm", *gnorm, stream)
                call(ga["out"][0], *ga["out"][1], stream)
                self._residual("w_out", lw["ln_post"], stream)
                gi += 1
            else:
                prep, attn = self._attn_args[ai]
                call(ga["qkv"][0], *ga["qkv"][1], stream)
                if self.splits["w_qkv"]:
                    call("dflash_splitk_reduce", self.part.data_ptr(), self.splits["w_qkv"], M,
                         cfg.attn_proj_rows, self.aproj.data_ptr(), cfg.attn_proj_rows, stream)
                call("dflash_attn_prep", *prep, stream)
                call("dflash_attn_verify", *attn, stream)
                call(ga["o"][0], *ga["o"][1], stream)
                self._residual("w_o", lw["ln_post"], stream)
                ai += 1
            call(ga["gu"][0], *ga["gu"][1], stream)
            call(ga["down"][0], *ga["down"][1], stream)
        self._residual("w_down", self.w.final_norm, stream)
        call(self._lm_fn, *self._lm_args, stream)

    def _forward_accept_hipblaslt(self):
        cfg, B, T = self.cfg, self.B, self.T
        stream = _lib.stream_handle(self.device)
        call = _lib.call
        M, H, I = B * T, cfg.hidden_size, cfg.intermediate_size
        eps = float(cfg.rms_norm_eps)
        torch.index_select(self.w.embed, 0, self.tokens.view(-1), out=self.h)
        r = None
        gi = ai = 0
        for i in range(cfg.num_hidden_layers):
            lw = self.w.layers[i]
            call("dflash_add_rmsnorm", self.h.data_ptr(), None if r is None else r.data_ptr(),
                 lw["ln_in"].data_ptr(), self.h.data_ptr(), self.xn.data_ptr(), M, H, eps, stream)
            if cfg.is_linear(i):
                prologue, scan, gnorm, _ = self._gdn_args[gi]
                self._mm(self.xn, lw["w_in"], self.proj[gi])
                call("dflash_gdn_prologue", *prologue, stream)
                call("dflash_gdn_verify_scan_rollback", *scan, stream)
                call("dflash_gdn_gated_rmsnorm", *gnorm, stream)
                self._mm(self.gnorm.view(M, -1), lw["w_out"], self.r)
                gi += 1
            else:
                prep, attn = self._attn_args[ai]
                self._mm(self.xn, lw["w_qkv"], self.aproj)
                call("dflash_attn_prep", *prep, stream)
                call("dflash_attn_verify", *attn, stream)
                self._mm(self.attn_out, lw["w_o"], self.r)
                ai += 1
            r = self.r
            call("dflash_add_rmsnorm", self.h.data_ptr(), r.data_ptr(), lw["ln_post"].data_ptr(),
                 self.h.data_ptr(), self.xn.data_ptr(), M, H, eps, stream)
            self._mm(self.xn, lw["w_gu"], self.gu)
            call("dflash_swiglu", self.gu.data_ptr(), self.mlp_act.data_ptr(), M, I, stream)
            self._mm(self.mlp_act, lw["w_down"], self.r)
        call("dflash_add_rmsnorm", self.h.data_ptr(), self.r.data_ptr(), self.w.final_norm.data_ptr(),
             self.h.data_ptr(), self.xn.data_ptr(), M, H, eps, stream)
        call(self._lm_fn, *self._lm_args, stream)

    def commit(self):
        """keep = matched + 1, lens += keep, and every conv window rolled to
        keep tokens (the recurrent states follow on the next step's load)."""
        cfg, lc, B, T = self.cfg, self.cfg.linear, self.B, self.T
        stream = _lib.stream_handle(self.device)
        _lib.call("dflash_commit_accept", self.matched.data_ptr(), self.keep.data_ptr(),
                  self.lens.data_ptr(), B, T, stream)
        rows = cfg.in_proj_rows
        cin, qkv, cout = self._conv_ptrs
        _lib.call("dflash_conv_rollback", cin, qkv, cout, self.keep.data_ptr(), cfg.n_linear, B, T,
                  lc.linear_conv_kernel_dim - 1, lc.conv_dim, T * rows, rows, 2, stream)

    def step(self):
        self.forward_accept()
        self.commit()

    # ------------------------------------------------------------- HIP graph
    def capture_step(self):
        """Capture one step (forward, accept, commit) as a HIP graph.  The
        capture itself does not execute the step."""
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

    def logits(self):
        """The LM-head logits of the last forward (a plain GEMM; for tests)."""
        return torch.nn.functional.linear(self.xn, self.w.lm_head).float().view(self.B, self.T, -1)
