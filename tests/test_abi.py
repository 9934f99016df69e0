"""The C-ABI library: loads, exports every declared entry point, and rejects
bad arguments before any launch (runs without a GPU: nothing here computes)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "dflash_gdn.h"


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dflash_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from dflash_mlx import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail("libdflash_gfx950.so is not built; run __graft_entry__.build()")
    return _lib.load()


def test_header_declares_expected_entry_points():
    names = _declared_functions()
    assert names == sorted([
        "dflash_abi_version", "dflash_strerror", "dflash_gdn_verify_scan",
        "dflash_gdn_verify_scan_rollback", "dflash_gdn_replay",
        "dflash_greedy_accept_workspace_bytes", "dflash_greedy_accept", "dflash_tape_select",
        "dflash_greedy_accept_noalloc_max_bytes", "dflash_greedy_accept_noalloc",
        "dflash_conv_rollback", "dflash_lm_head_accept_workspace_bytes",
        "dflash_lm_head_greedy_accept", "dflash_gdn_prologue", "dflash_gdn_gated_rmsnorm",
        "dflash_gdn_prologue_scan_rollback", "dflash_lm_head_greedy_accept_tiled",
        "dflash_greedy_accept_conv_rollback", "dflash_gdn_verify_scan_rollback_argmax",
        "dflash_accept_keys_conv_rollback",
        "dflash_gdn_verify_step_workspace_bytes", "dflash_gdn_verify_step",
        "dflash_gdn_chunked_prefill_workspace_bytes", "dflash_gdn_chunked_prefill",
        "dflash_add_rmsnorm", "dflash_swiglu", "dflash_attn_prep",
        "dflash_attn_verify_workspace_bytes", "dflash_attn_verify", "dflash_commit_accept",
        "dflash_add_rmsnorm_splitk", "dflash_add_rmsnorm_capture", "dflash_embed_rmsnorm", "dflash_gemm_bf16", "dflash_gemm_splits",
        "dflash_splitk_reduce", "dflash_splitk_swiglu_reduce", "dflash_gemm_bf16_swiglu",
        "dflash_weight_tile_bytes",
        "dflash_weight_tile_bf16", "dflash_gemm_bf16_tiled", "dflash_gemm_bf16_swiglu_tiled",
        "dflash_gemm_tail_workspace_bytes",
        "dflash_gemm_bf16_tiled_residual_norm",
        "dflash_gemm_bf16_tiled_normed", "dflash_gemm_bf16_swiglu_tiled_normed",
        "dflash_gemm_bf16_tiled_prefill", "dflash_gemm_bf16_swiglu_tiled_prefill",
        "dflash_gemm_bf16_tiled_prefill_splitk", "dflash_gemm_bf16_tiled_prefill_rows",
        "dflash_attn_prefill",
    ])


def test_library_exports_every_declared_symbol(lib):
    from dflash_mlx import _lib

    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_library_targets_gfx950_only():
    from dflash_mlx import _lib

    blob = _lib.LIB_PATH.read_bytes()
    assert b"gfx950" in blob
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert other not in blob


def test_abi_version_and_strerror(lib):
    assert lib.dflash_abi_version() == 4
    assert lib.dflash_strerror(0) == b"ok"
    assert b"NULL" in lib.dflash_strerror(-1)
    assert lib.dflash_strerror(-999) == b"unknown dflash error"


def test_scan_validation_codes(lib):
    f = lib.dflash_gdn_verify_scan
    dummy = ctypes.c_void_p(0x1000)
    # missing k
    assert f(None, None, dummy, dummy, dummy, dummy, None, dummy, None, None,
             1, 16, 4, 4, 64, 64, None, None) == -1
    # q without out
    assert f(dummy, dummy, dummy, dummy, dummy, dummy, None, dummy, None, None,
             1, 16, 4, 4, 64, 64, None, None) == -1
    # Hv not a multiple of Hk
    assert f(dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, None, None,
             1, 16, 3, 4, 64, 64, None, None) == -2
    # unsupported Dk
    assert f(dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, None, None,
             1, 16, 4, 4, 80, 64, None, None) == -3
    # Dv not a multiple of 16
    assert f(dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, None, None,
             1, 16, 4, 4, 64, 40, None, None) == -3
    # misaligned k pointer
    odd = ctypes.c_void_p(0x1002)
    assert f(dummy, odd, dummy, dummy, dummy, dummy, dummy, dummy, None, None,
             1, 16, 4, 4, 64, 64, None, None) == -4


def test_accept_workspace_and_validation(lib):
    ws = lib.dflash_greedy_accept_workspace_bytes(1, 16, 151936)
    assert ws > 0 and ws % 8 == 0
    assert lib.dflash_greedy_accept_workspace_bytes(0, 16, 10) == 0
    dummy = ctypes.c_void_p(0x1000)
    f = lib.dflash_greedy_accept
    # too-small workspace
    assert f(dummy, 0, 16 * 1024, 1024, None, 0, 0, dummy, dummy, dummy,
             1, 16, 1024, dummy, 8, None) == -5
    # bad dtype
    assert f(dummy, 7, 16 * 1024, 1024, None, 0, 0, dummy, dummy, dummy,
             1, 16, 1024, dummy, 1 << 20, None) == -3
    # draft missing while n_draft > 0
    assert f(dummy, 0, 16 * 1024, 1024, None, 16, 16, dummy, dummy, dummy,
             1, 16, 1024, dummy, 1 << 20, None) == -1


def test_rollback_validation(lib):
    f = lib.dflash_tape_select
    assert f(None, None, None, None, 0, 1, 16, 10, 0, None) == 0  # nothing to do
    assert f(None, None, None, None, 1, 1, 16, 10, 0, None) == -1
    assert f(None, None, None, None, 1, 1, 16, 10, -4, None) == -2
    g = lib.dflash_conv_rollback
    assert g(None, None, None, None, 1, 1, 16, 9, 8192, 0, 0, 2, None) == -3  # K1 > 8
    assert g(None, None, None, None, 1, 1, 16, 3, 8192, 0, 0, 3, None) == -3  # elem size


def test_ops_refuse_cpu_tensors():
    """No CPU fallback: host tensors are rejected, not computed."""
    import torch

    from dflash_mlx import gated_delta_verify, greedy_accept

    q = torch.zeros(1, 2, 1, 64, dtype=torch.bfloat16)
    v = torch.zeros(1, 2, 1, 64, dtype=torch.bfloat16)
    g = torch.zeros(1, 2, 1)
    s = torch.zeros(1, 1, 64, 64)
    with pytest.raises(ValueError, match="ROCm device"):
        gated_delta_verify(q, q, v, g, g, s)
    with pytest.raises(ValueError, match="ROCm device"):
        greedy_accept(torch.zeros(1, 2, 8), None)


def test_model_op_size_limits(lib):
    """Shapes whose row or grid counts overflow int are refused before any launch."""
    d = ctypes.c_void_p(0x1000)
    big = 1 << 16
    # gated RMSNorm: B*T*H rows > 2^31 - 1
    assert lib.dflash_gdn_gated_rmsnorm(d, d, None, d, d, big, big, 32, 128, 1e-6, None) == -2
    # prologue: B*T workgroup rows > 2^31 - 1
    assert lib.dflash_gdn_prologue(d, 0, 0, d, d, d, d, None, d, d, d, d, d, d,
                                   big, big, 4, 16, 32, 128, 128, 1e-6, None) == -2
    # attention prep: B*T workgroups > 2^31 - 1
    assert lib.dflash_attn_prep(d, 5120, d, d, d, d, d, d, None, big, big, 16, 4, 128, 4096,
                                64, 1e7, 1e-6, None) == -2
    # attention: B beyond the partial kernel's grid.z
    assert lib.dflash_attn_verify(d, d, d, d, d, 4096, d, 70000, 16, 16, 4, 128, 4096, 4096,
                                  0.0884, d, 1 << 40, None) == -2


def test_scan_with_argmax_and_keys_accept_validation(lib):
    """The scan launch carrying the accept's argmax, and the accept + conv
    rollback from those keys, refuse bad arguments before any launch."""
    d = ctypes.c_void_p(0x1000)
    f = lib.dflash_gdn_verify_scan_rollback_argmax
    ws = lib.dflash_greedy_accept_workspace_bytes(1, 16, 1024)

    def scan(logits=d, dtype=0, B_acc=1, N=16, V=1024, work=d, wsb=ws, B=1, T=16):
        return f(d, d, d, d, d, d, d, d, 16, 1, d, None, d, B, T, 4, 4, 64, 64, None,
                 logits, dtype, 16 * 1024, 1024, B_acc, N, V, work, wsb, None)

    assert scan(B_acc=0) == -2                  # no accept rows
    assert scan(B_acc=2048, N=16) == -2         # more than 16384 logits rows
    assert scan(T=0) == -2                      # the launch must have scan work
    assert scan(logits=None) == -1
    assert scan(work=None) == -1
    assert scan(dtype=2) == -3                  # fp16 logits: not in this launch
    assert scan(wsb=ws - 8) == -5               # workspace too small
    assert scan(logits=ctypes.c_void_p(0x1008)) == -4   # rows not 16-byte aligned
    # final_state aliasing the state buffer
    assert f(d, d, d, d, d, d, d, d, 16, 1, d, d, d, 1, 16, 4, 4, 64, 64, None,
             d, 0, 16 * 1024, 1024, 1, 16, 1024, d, ws, None) == -2
    g = lib.dflash_accept_keys_conv_rollback

    def keys(draft=d, n_draft=15, work=d, wsb=ws, K1=3, elem=2, N=16):
        return g(draft, 16, n_draft, d, d, d, 1, N, 1024, work, wsb, d, d, d, 1, d, 1, 16, K1,
                 8192, 16 * 8192, 8192, elem, None)

    assert keys(draft=None) == -1               # drafts missing while n_draft > 0
    assert keys(work=None) == -1
    assert keys(wsb=8) == -5
    assert keys(K1=9) == -3                     # more window rows than one lane holds
    assert keys(elem=3) == -3
    assert keys(N=0) == -2


def test_verify_step_validation(lib):
    """The single-launch verify step refuses, before any launch: more accept
    rows than one finishing workgroup holds (N > 64), more window rows than
    it copies (K1 > 4), more layers than one launch's tables (L > 32), the
    next keep buffer equal to the one the scan reads, a workspace off a
    256-byte boundary, and conv rows that are not whole 16-byte units."""
    d = ctypes.c_void_p(0x1000)
    keep_in, keep_out = ctypes.c_void_p(0x3000), ctypes.c_void_p(0x4000)
    f = lib.dflash_gdn_verify_step
    ws = lib.dflash_gdn_verify_step_workspace_bytes(1, 16, 1024)
    assert ws > 0

    def step(N=16, K1=3, L=1, out_keep=keep_out, work=ctypes.c_void_p(0x100000), C=8192):
        tab = (ctypes.c_void_p * max(L, 1))(*([0x1000] * max(L, 1)))
        return f(d, d, d, d, d, d, d, keep_in, 16, 1, d, None, d, 1, 16, 4, 4, 64, 64, None,
                 d, 0, 16 * 1024, 1024, 1, N, 1024,
                 d, 16, 15, d, d, d, 1, out_keep,
                 tab, tab, tab, L, K1, C, 16 * C, C,
                 work, ws * 8, None)

    assert step(N=65) == -3
    assert step(K1=5) == -3
    assert step(L=33) == -3
    assert step(out_keep=keep_in) == -2
    assert step(work=ctypes.c_void_p(0x100008)) == -4
    assert step(C=8190) == -4          # 16 380-byte rows: not 16-byte units
    assert step(out_keep=None) == -1


def test_gemm_tail_workspace_and_normed_validation(lib):
    """The tiled GEMMs' tail-split workspace must hold
    dflash_gemm_tail_workspace_bytes() bytes on a 256-byte boundary; the
    normed forms take K <= 16384 (their LDS copy of the norm weight)."""
    d = ctypes.c_void_p(0x1000)
    tail = lib.dflash_gemm_tail_workspace_bytes()
    assert tail > 1024
    aligned, odd = ctypes.c_void_p(0x200000), ctypes.c_void_p(0x200080)
    tiled = lib.dflash_gemm_bf16_tiled
    assert tiled(d, 2560, d, d, 2560, 16, 2560, 2560, 1, 32, 4, aligned, tail - 1, None) == -5
    assert tiled(d, 2560, d, d, 2560, 16, 2560, 2560, 1, 32, 4, odd, tail, None) == -4
    sw = lib.dflash_gemm_bf16_swiglu_tiled
    assert sw(d, 2560, d, d, 9216, 16, 18432, 2560, 4, aligned, tail - 1, None) == -5
    assert sw(d, 2560, d, d, 9216, 16, 18432, 2560, 4, odd, tail, None) == -4
    normed = lib.dflash_gemm_bf16_tiled_normed
    assert normed(d, 2560, d, d, 160, 1e-6, None, d, d, 2560, 16, 2560, 2560, 1, 32, 4,
                  aligned, tail - 1, None) == -5
    assert normed(d, 20480, d, d, 160, 1e-6, None, d, d, 2560, 16, 2560, 20480, 1, 32, 4,
                  aligned, tail, None) == -2
    sw_normed = lib.dflash_gemm_bf16_swiglu_tiled_normed
    assert sw_normed(d, 2560, d, d, 160, 1e-6, None, d, d, 9216, 16, 18432, 2560, 4,
                     odd, tail, None) == -4
    assert sw_normed(d, 20480, d, d, 160, 1e-6, None, d, d, 9216, 16, 18432, 20480, 4,
                     aligned, tail, None) == -2


def test_splitk_swiglu_reduce_validation(lib):
    """The gated reduce over the w_pairs column order: N a multiple of 32, at
    least one split, 16-byte aligned partials, output rows of at least N/2
    columns in 8-byte pieces; M = 0 is a no-op."""
    d = ctypes.c_void_p(0x1000)
    f = lib.dflash_splitk_swiglu_reduce
    assert f(d, 2, 0, 64, d, 32, None) == 0
    assert f(d, 2, 16, 48, d, 24, None) == -2      # N % 32
    assert f(d, 0, 16, 64, d, 32, None) == -2      # nsplit < 1
    assert f(None, 2, 16, 64, d, 32, None) == -1
    assert f(d, 2, 16, 64, None, 32, None) == -1
    assert f(ctypes.c_void_p(0x1008), 2, 16, 64, d, 32, None) == -4
    assert f(d, 2, 16, 64, ctypes.c_void_p(0x1004), 32, None) == -4
    assert f(d, 2, 16, 64, d, 30, None) == -4      # stride % 4
    assert f(d, 2, 16, 64, d, 28, None) == -4      # rows shorter than N/2


def test_prefill_gemm_validation(lib):
    """The prompt-sized GEMMs refuse shapes the fragment layout cannot hold
    and misaligned rows before any launch; M = 0 is a no-op."""
    d = ctypes.c_void_p(0x1000)
    f = lib.dflash_gemm_bf16_tiled_prefill
    assert f(d, 2560, d, d, 2560, 0, 2560, 2560, None) == 0
    assert f(d, 2560, d, d, 2560, 100, 2568, 2560, None) == -2     # N % 16
    assert f(d, 2560, d, d, 2560, 100, 2560, 2592, None) == -2     # K % 64
    assert f(d, 2000, d, d, 2560, 100, 2560, 2560, None) == -2     # x rows shorter than K
    assert f(d, 2560, d, d, 2000, 100, 2560, 2560, None) == -2     # out rows shorter than N
    assert f(None, 2560, d, d, 2560, 100, 2560, 2560, None) == -1
    assert f(ctypes.c_void_p(0x1008), 2560, d, d, 2560, 100, 2560, 2560, None) == -4
    assert f(d, 2564, d, d, 2560, 100, 2560, 2560, None) == -4     # x stride % 8
    assert f(d, (1 << 22) + 8, d, d, 2560, 100, 2560, 2560, None) == -2  # x stride > 2^22
    assert f(d, 2560, d, ctypes.c_void_p(0x1004), 2560, 100, 2560, 2560, None) == -4
    h = lib.dflash_gemm_bf16_tiled_prefill_splitk
    assert h(d, 2560, d, d, 0, 100, 2560, 2560, None) == -2       # nsplit < 1
    assert h(d, 2560, d, None, 3, 100, 2560, 2560, None) == -1
    assert h(d, 2560, d, ctypes.c_void_p(0x1008), 3, 100, 2560, 2560, None) == -4
    g = lib.dflash_gemm_bf16_swiglu_tiled_prefill
    assert g(d, 2560, d, d, 9216, 100, 18448, 2560, None) == -2   # N % 32
    assert g(d, 2560, d, d, 9000, 100, 18432, 2560, None) == -2   # out rows shorter than N/2
    assert g(d, 2560, d, d, 9218, 100, 18432, 2560, None) == -4   # out stride % 4


def test_prefill_gemm_rows_validation(lib):
    """A row range of a tiled weight: row0 and N whole 16-row tiles (32 with
    the gated form), inside the weight; partials and the gated form are
    exclusive; otherwise the whole-weight checks."""
    d = ctypes.c_void_p(0x1000)
    f = lib.dflash_gemm_bf16_tiled_prefill_rows
    assert f(d, 2560, d, 4096, 256, d, 256, None, 0, 0, 256, 2560, 0, None) == 0     # M = 0
    assert f(d, 2560, d, 4096, 8, d, 256, None, 0, 100, 256, 2560, 0, None) == -2    # row0 % 16
    assert f(d, 2560, d, 4096, 16, d, 128, None, 0, 100, 256, 2560, 1, None) == -2   # row0 % 32
    assert f(d, 2560, d, 4096, 3968, d, 256, None, 0, 100, 256, 2560, 0, None) == -2  # past w_rows
    assert f(d, 2560, d, 4100, 0, d, 256, None, 0, 100, 256, 2560, 0, None) == -2    # w_rows % 16
    assert f(d, 2560, d, 4096, -16, d, 256, None, 0, 100, 256, 2560, 0, None) == -2  # row0 < 0
    assert f(d, 2560, d, 4096, 0, None, 0, d, 2, 100, 256, 2560, 1, None) == -2     # partials + gated
    assert f(d, 2560, d, 4096, 0, None, 0, None, 2, 100, 256, 2560, 0, None) == -1
    assert f(d, 2560, d, 4096, 0, d, 200, None, 0, 100, 256, 2560, 0, None) == -2    # out rows < N


def test_attn_prefill_validation(lib):
    d = ctypes.c_void_p(0x1000)
    f = lib.dflash_attn_prefill
    assert f(d, d, d, d, d, 5120, d, 16, 16, 4, 64, 4096, 0.09, None) == -3    # D != 128
    assert f(d, d, d, d, d, 5120, d, 16, 20, 4, 128, 4096, 0.09, None) == -2   # Hq % Hkv
    assert f(d, d, d, d, d, 5120, d, 16, 16, 2, 128, 4096, 0.09, None) == -2   # Hq / Hkv > 4
    assert f(d, d, d, d, d, 5120, d, 16, 16, 4, 128, 4000, 0.09, None) == -2   # Smax % 64
    assert f(d, d, d, d, d, 100, d, 16, 16, 4, 128, 4096, 0.09, None) == -2    # gate stride
    assert f(d, d, d, None, d, 5120, d, 16, 16, 4, 128, 4096, 0.09, None) == -1
    assert f(d, ctypes.c_void_p(0x1008), d, d, d, 5120, d, 16, 16, 4, 128, 4096, 0.09,
             None) == -4
    assert f(None, None, None, None, None, 5120, None, 0, 16, 4, 128, 4096, 0.09, None) == 0


def test_noalloc_refuses_shapes_beyond_its_array_before_any_device_call(lib):
    """dflash_greedy_accept_noalloc refuses key arrays beyond its 1 MiB static
    array from the shapes alone, before touching a device (no GPU here)."""
    d = ctypes.c_void_p(0x1000)
    assert lib.dflash_greedy_accept_noalloc_max_bytes() == 1 << 20
    B, N, V = 8193, 16, 4096  # 131088 rows -> 1 MiB + 128 B of keys
    assert lib.dflash_greedy_accept_noalloc(d, 0, N * V, V, None, 0, 0, d, None, None, B, N, V,
                                            None) == -5
