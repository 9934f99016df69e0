"""GPU parity of the prompt-sized GEMMs (dflash_gemm_bf16_tiled_prefill,
dflash_gemm_bf16_swiglu_tiled_prefill) over the fragment-tiled weights.

* Against an fp32 torch reference of the same bf16 inputs: out within one
  bf16 rounding of the reference (|err| <= 2^-8 |ref| + 1e-3 * rms(ref)); the
  gated form against silu(x.G^T) * (x.U^T) in fp32 with the same bound.
* Bit for bit against the verify-sized tiled GEMM with one wave per k-range
  and one split (dflash_gemm_bf16_tiled, k_waves 1, nsplit 1): both keep one
  fp32 chain per output over the k-steps in order, so at M <= 64 their sums
  are the same bits — a check that pins the k-slot order of the activation
  operand, which the fp32 bound would not catch at small K.
* The two workgroup tiles (256 x 256 when its units fill the device, else
  256 x 128) bit for bit against each other: a launch over M rows against
  launches over 128-row slices of the same rows, which take the other tile.
Shapes: every projection of the config-c4 layers at prompt lengths, M and N
tails (M not a multiple of 128 or 256, N not a multiple of 256, down to a
last weight tile of one 16-row tile), K = 64.
"""
from __future__ import annotations

import pytest
import torch

from dflash_mlx import _lib

pytestmark = pytest.mark.gpu

C4_PROJ = [(12352, 2560), (2560, 4096), (5120, 2560), (2560, 2048), (2560, 9216)]


def _tile(w, device):
    n, k = w.shape
    lib = _lib.load()
    t = torch.empty(int(lib.dflash_weight_tile_bytes(n, k)) // 2, dtype=torch.bfloat16,
                    device=device)
    _lib.call("dflash_weight_tile_bf16", w.data_ptr(), w.stride(0), t.data_ptr(), n, k,
              _lib.stream_handle(device))
    return t


def _inputs(device, M, N, K, seed):
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=device).bfloat16()
    w = (0.02 * torch.randn(N, K, generator=g, device=device)).bfloat16()
    return x, w


def _prefill(device, x, wt, M, N, K, swiglu=False):
    n_out = N // 2 if swiglu else N
    out = torch.full((M, n_out), float("nan"), dtype=torch.bfloat16, device=device)
    name = "dflash_gemm_bf16_swiglu_tiled_prefill" if swiglu else "dflash_gemm_bf16_tiled_prefill"
    _lib.call(name, x.data_ptr(), x.stride(0), wt.data_ptr(), out.data_ptr(), out.stride(0), M, N,
              K, _lib.stream_handle(device))
    torch.cuda.synchronize()
    return out


def _check(out, ref):
    scale = ref.pow(2).mean().sqrt().item()
    assert torch.isfinite(out).all()
    err = ((out.float() - ref).abs() - (2 ** -8) * ref.abs()).max().item()
    assert err <= 1e-3 * scale, (err, scale)


@pytest.mark.parametrize("M,N,K", [(1, 16, 64), (17, 272, 128), (128, 256, 64),
                                   (300, 1040, 640), (129, 4112, 192), (1000, 48, 2560)])
def test_prefill_gemm_ragged(device, M, N, K):
    print(f"[prefill gemm] M={M} N={N} K={K}", flush=True)
    x, w = _inputs(device, M, N, K, seed=M + 3 * N + K)
    out = _prefill(device, x, _tile(w, device), M, N, K)
    _check(out, x.float() @ w.float().t())


@pytest.mark.parametrize("N,K", C4_PROJ)
def test_prefill_gemm_c4_projections(device, N, K):
    M = 1100
    print(f"[prefill gemm] c4 projection M={M} N={N} K={K}", flush=True)
    x, w = _inputs(device, M, N, K, seed=N + K)
    out = _prefill(device, x, _tile(w, device), M, N, K)
    _check(out, x.float() @ w.float().t())


@pytest.mark.parametrize("M,N,K", [(16, 2560, 2560), (37, 1040, 640), (64, 18432, 256),
                                   (1, 16, 64)])
def test_prefill_gemm_matches_verify_gemm_bits(device, M, N, K):
    """The same bits as the verify-sized tiled GEMM with one k-range per wave
    and one split, which adds the same products in the same order."""
    print(f"[prefill gemm] vs verify gemm M={M} N={N} K={K}", flush=True)
    x, w = _inputs(device, M, N, K, seed=7 * M + N)
    wt = _tile(w, device)
    out = _prefill(device, x, wt, M, N, K)
    ref = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=device)
    _lib.call("dflash_gemm_bf16_tiled", x.data_ptr(), K, wt.data_ptr(), ref.data_ptr(), N, M, N, K,
              1, 16, 1, None, 0, _lib.stream_handle(device))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("M,N,K,swiglu", [(4000, 4112, 192, False), (4096, 12352, 128, False),
                                           (2900, 8224, 128, True), (4096, 5120, 256, False),
                                           (4096, 4096, 64, False)])
def test_prefill_gemm_wide_tile_matches_narrow_bits(device, M, N, K, swiglu):
    """The 256 x 256 tile (chosen here: its units reach the device's compute
    units) against the 256 x 128 tile (chosen for each 128-row slice alone):
    each output row depends on its own activation row only, so the slices
    must reproduce the whole launch bit for bit.  N = 4112 leaves one 16-row
    tile in the last weight tile (three of its four weight-row waves hold no
    rows), M = 4000 / 2900 a partial last activation tile."""
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    assert -(-N // 256) * -(-M // 256) >= cus and -(-N // 256) * 1 < cus
    print(f"[prefill gemm] wide vs narrow tile M={M} N={N} K={K} swiglu={swiglu}", flush=True)
    x, w = _inputs(device, M, N, K, seed=M + N + K)
    wt = _tile(w, device)
    whole = _prefill(device, x, wt, M, N, K, swiglu=swiglu)
    parts = torch.cat([_prefill(device, x[r:r + 128], wt, min(128, M - r), N, K, swiglu=swiglu)
                       for r in range(0, M, 128)])
    assert torch.equal(whole, parts)
    if not swiglu:
        _check(whole, x.float() @ w.float().t())


def test_prefill_gemm_wide_tile_one_short_block(device):
    """The 256 x 256 tile over fewer than 256 rows (200: its units take one
    round where the 256 x 128 tile's take two), so the activation loaders
    clamp rows 200-255 of the block: bit for bit the 128-row slices (the
    other tile) and within one bf16 rounding of fp32."""
    M, N, K = 200, 65536, 128
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    wide, narrow = -(-N // 256), -(-N // 256) * 2
    assert 10 * -(-wide // cus) <= 7 * -(-narrow // cus)
    print(f"[prefill gemm] wide tile, one short block M={M} N={N} K={K}", flush=True)
    x, w = _inputs(device, M, N, K, seed=7)
    wt = _tile(w, device)
    whole = _prefill(device, x, wt, M, N, K)
    parts = torch.cat([_prefill(device, x[r:r + 128], wt, min(128, M - r), N, K)
                       for r in range(0, M, 128)])
    assert torch.equal(whole, parts)
    _check(whole, x.float() @ w.float().t())


@pytest.mark.parametrize("M,I,K", [(300, 9216, 2560), (5, 16, 64), (129, 272, 192)])
def test_prefill_gemm_swiglu(device, M, I, K):
    """Gated form over the w_pairs layout (32-row blocks: 16 gate rows, then
    the 16 matching up rows)."""
    print(f"[prefill gemm] swiglu M={M} I={I} K={K}", flush=True)
    g = torch.Generator(device=device).manual_seed(M + I)
    x = torch.randn(M, K, generator=g, device=device).bfloat16()
    gate = (0.02 * torch.randn(I, K, generator=g, device=device)).bfloat16()
    up = (0.02 * torch.randn(I, K, generator=g, device=device)).bfloat16()
    pairs = torch.stack([gate.view(I // 16, 16, K), up.view(I // 16, 16, K)], 1).reshape(2 * I, K)
    out = _prefill(device, x, _tile(pairs.contiguous(), device), M, 2 * I, K, swiglu=True)
    gf, uf = x.float() @ gate.float().t(), x.float() @ up.float().t()
    _check(out, torch.nn.functional.silu(gf) * uf)
    # the same bits as the verify-sized gated GEMM at M <= 64 rows (one k-range per wave)
    if M <= 64:
        wt = _tile(pairs.contiguous(), device)
        ref = torch.full((M, I), float("nan"), dtype=torch.bfloat16, device=device)
        _lib.call("dflash_gemm_bf16_swiglu_tiled", x.data_ptr(), K, wt.data_ptr(), ref.data_ptr(),
                  I, M, 2 * I, K, 1, None, 0, _lib.stream_handle(device))
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


@pytest.mark.parametrize("M,N,K,ns,swiglu", [(128, 12352, 2560, 4, False), (37, 5120, 2560, 3, False),
                                              (128, 18432, 2560, 3, True), (5, 96, 192, 2, True),
                                              (300, 2080, 640, 4, True)])
def test_prefill_splitk_reduce_matches_one_launch(device, M, N, K, ns, swiglu):
    """The prompt pass's split form of a bf16 projection: split-K partials
    summed and cast by dflash_splitk_reduce (gated: dflash_splitk_swiglu_reduce
    over the w_pairs columns) against the one-launch GEMM: both round fp32
    sums of the same products added in another order, so they sit within one
    bf16 ulp (2^-7 relative) of each other (two for the gated form) plus
    1e-4 of the output scale; the gated form also against the fp32
    reference."""
    print(f"[prefill gemm] split-K + reduce M={M} N={N} K={K} nsplit={ns} swiglu={swiglu}",
          flush=True)
    x, w = _inputs(device, M, N, K, seed=M * 5 + N + ns)
    wt = _tile(w, device)
    one = _prefill(device, x, wt, M, N, K, swiglu=swiglu)
    lib = _lib.load()
    used = int(lib.dflash_gemm_splits(K, ns))
    part = torch.full((used, M, N), float("nan"), device=device)
    _lib.call("dflash_gemm_bf16_tiled_prefill_splitk", x.data_ptr(), K, wt.data_ptr(),
              part.data_ptr(), ns, M, N, K, _lib.stream_handle(device))
    n_out = N // 2 if swiglu else N
    ow = torch.full((M, n_out + 8), float("nan"), dtype=torch.bfloat16, device=device)
    _lib.call("dflash_splitk_swiglu_reduce" if swiglu else "dflash_splitk_reduce", part.data_ptr(),
              used, M, N, ow.data_ptr(), n_out + 8, _lib.stream_handle(device))
    torch.cuda.synchronize()
    got = ow[:, :n_out]
    assert torch.isnan(ow[:, n_out:].float()).all()  # nothing past the row written
    ref = one.float()
    tol = (2 if swiglu else 1) * (2 ** -7) * ref.abs() + 1e-4 * ref.pow(2).mean().sqrt()
    assert ((got.float() - ref).abs() <= tol).all()
    if swiglu:
        g_ = x.float() @ w.float().t()
        pairs = g_.view(M, N // 32, 2, 16)
        _check(got, (torch.nn.functional.silu(pairs[:, :, 0]) * pairs[:, :, 1]).reshape(M, N // 2))


@pytest.mark.parametrize("M,N,K,row0,rows,swiglu,ns", [
    (300, 4112, 192, 256, 3856, False, 0), (300, 4112, 192, 4096, 16, False, 3),
    (129, 2080, 640, 0, 1024, True, 0), (129, 2080, 640, 1024, 1056, False, 4),
    (1000, 12352, 256, 12288, 64, False, 4)])
def test_prefill_gemm_row_range(device, M, N, K, row0, rows, swiglu, ns):
    """dflash_gemm_bf16_tiled_prefill_rows over rows row0 .. row0+rows-1 of a
    tiled weight: bf16 (or gated) outputs bit for bit the same columns of the
    whole-weight launch; split-K partials summing to those columns' fp32
    reference, and through the reduce (the gated one for a w_pairs range)
    within one bf16 ulp of the whole launch's columns."""
    print(f"[prefill gemm] rows {row0}..{row0 + rows} of {N} M={M} K={K} swiglu={swiglu} "
          f"nsplit={ns}", flush=True)
    x, w = _inputs(device, M, N, K, seed=M + row0 + rows)
    wt = _tile(w, device)
    gated = swiglu or (ns > 0 and row0 % 32 == 0 and rows % 32 == 0 and N % 32 == 0)
    whole = _prefill(device, x, wt, M, N, K, swiglu=swiglu)
    st = _lib.stream_handle(device)
    if ns == 0:
        n_out = rows // 2 if swiglu else rows
        got = torch.full((M, n_out), float("nan"), dtype=torch.bfloat16, device=device)
        _lib.call("dflash_gemm_bf16_tiled_prefill_rows", x.data_ptr(), K, wt.data_ptr(), N, row0,
                  got.data_ptr(), n_out, None, 0, M, rows, K, int(swiglu), st)
        torch.cuda.synchronize()
        c0 = row0 // 2 if swiglu else row0
        assert torch.equal(got, whole[:, c0:c0 + n_out])
        return
    used = int(_lib.load().dflash_gemm_splits(K, ns))
    part = torch.full((used, M, rows), float("nan"), device=device)
    _lib.call("dflash_gemm_bf16_tiled_prefill_rows", x.data_ptr(), K, wt.data_ptr(), N, row0,
              None, 0, part.data_ptr(), ns, M, rows, K, 0, st)
    torch.cuda.synchronize()
    ref = x.float() @ w[row0:row0 + rows].float().t()
    scale = ref.pow(2).mean().sqrt().item()
    assert torch.isfinite(part).all()
    assert (part.sum(0) - ref).abs().max().item() <= 1e-4 * scale + 1e-5
    red = torch.full((M, rows), float("nan"), dtype=torch.bfloat16, device=device)
    _lib.call("dflash_splitk_reduce", part.data_ptr(), used, M, rows, red.data_ptr(), rows, st)
    torch.cuda.synchronize()
    one = whole[:, row0:row0 + rows].float()
    assert ((red.float() - one).abs() <= (2 ** -7) * one.abs() + 1e-4 * scale).all()
    if gated:  # the same range of a w_pairs weight through the gated reduce
        gw = _prefill(device, x, wt, M, N, K, swiglu=True)
        gr = torch.full((M, rows // 2), float("nan"), dtype=torch.bfloat16, device=device)
        _lib.call("dflash_splitk_swiglu_reduce", part.data_ptr(), used, M, rows, gr.data_ptr(),
                  rows // 2, st)
        torch.cuda.synchronize()
        g1 = gw[:, row0 // 2:(row0 + rows) // 2].float()
        gs = g1.pow(2).mean().sqrt().item()
        assert ((gr.float() - g1).abs() <= 2 * (2 ** -7) * g1.abs() + 1e-4 * gs).all()


@pytest.mark.parametrize("M,N,K", [(200, 528, 320), (2100, 8224, 320)])
def test_prefill_gemm_strided_rows(device, M, N, K):
    """Activation and output rows with strides larger than K and N (views
    into wider buffers), on the 256 x 128 tile (200 rows) and the 256 x 256
    tile (2100 rows: 297 units), whose activation loads take whole rows at
    the row stride."""
    print(f"[prefill gemm] strided rows M={M} N={N} K={K}", flush=True)
    x, w = _inputs(device, M, N, K, seed=11 + M)
    xw = torch.zeros(M, K + 64, dtype=torch.bfloat16, device=device)
    xw[:, 8:8 + K] = x
    xv = xw[:, 8:8 + K]
    wt = _tile(w, device)
    ow = torch.full((M, N + 12), float("nan"), dtype=torch.bfloat16, device=device)
    ov = ow[:, 4:4 + N]
    _lib.call("dflash_gemm_bf16_tiled_prefill", xv.data_ptr(), xv.stride(0), wt.data_ptr(),
              ov.data_ptr(), ov.stride(0), M, N, K, _lib.stream_handle(device))
    torch.cuda.synchronize()
    _check(ov, x.float() @ w.float().t())
    assert torch.isnan(ow[:, :4].float()).all() and torch.isnan(ow[:, 4 + N:].float()).all()


@pytest.mark.parametrize("M,N,K,ns", [(4096, 2560, 2048, 3), (300, 272, 640, 4), (17, 16, 64, 2),
                                      (4096, 2560, 192, 3), (4000, 2560, 384, 2)])
def test_prefill_gemm_splitk(device, M, N, K, ns):
    """Split-K partial sums: dflash_gemm_splits(K, ns) slots, every one
    written, summing to the fp32 reference within 1e-4 of its scale."""
    print(f"[prefill gemm] split-K M={M} N={N} K={K} nsplit={ns}", flush=True)
    x, w = _inputs(device, M, N, K, seed=M + N + ns)
    wt = _tile(w, device)
    used = int(_lib.load().dflash_gemm_splits(K, ns))
    part = torch.full((used, M, N), float("nan"), device=device)
    _lib.call("dflash_gemm_bf16_tiled_prefill_splitk", x.data_ptr(), K, wt.data_ptr(),
              part.data_ptr(), ns, M, N, K, _lib.stream_handle(device))
    torch.cuda.synchronize()
    assert torch.isfinite(part).all()
    ref = x.float() @ w.float().t()
    scale = ref.pow(2).mean().sqrt().item()
    assert (part.sum(0) - ref).abs().max().item() <= 1e-4 * scale + 1e-5
