"""ctypes binding of libdflash_gfx950.so (declared in include/dflash_gdn.h).

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch already loaded (both use the soname libamdhip64.so.7); loading
it first would pull in a second runtime whose streams torch does not know.

There is no fallback: if the library is missing or fails to load, every op
raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see above)

LIB_PATH = Path(__file__).resolve().parent / "libdflash_gfx950.so"

DFLASH_DTYPE_F32 = 0
DFLASH_DTYPE_BF16 = 1
DFLASH_DTYPE_F16 = 2

# Every entry point of include/dflash_gdn.h, with its ctypes signature.
_VP = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "dflash_abi_version": (_I, []),
    "dflash_strerror": (ctypes.c_char_p, [_I]),
    "dflash_gdn_verify_scan": (
        _I,
        [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I, _VP, _VP],
    ),
    "dflash_gdn_verify_scan_rollback": (
        _I,
        [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I,
         _VP, _VP],
    ),
    "dflash_gdn_verify_scan_rollback_argmax": (
        _I,
        [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I,
         _VP, _VP, _I, _I64, _I64, _I, _I, _I, _VP, _SZ, _VP],
    ),
    "dflash_gdn_verify_step_workspace_bytes": (_SZ, [_I, _I, _I]),
    "dflash_gdn_verify_step": (
        _I,
        [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I,
         _VP, _VP, _I, _I64, _I64, _I, _I, _I,  # scan, logits
         _VP, _I64, _I, _VP, _VP, _VP, _I, _VP,  # accept
         _VP, _VP, _VP, _I, _I, _I64, _I64, _I64,  # conv windows
         _VP, _SZ, _VP],
    ),
    "dflash_gdn_replay": (
        _I,
        [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I, _VP, _VP],
    ),
    "dflash_gdn_chunked_prefill_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "dflash_gdn_chunked_prefill": (
        _I,
        [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I, _VP, _VP, _SZ, _VP],
    ),
    "dflash_add_rmsnorm": (_I, [_VP, _VP, _VP, _VP, _VP, _I, _I, ctypes.c_float, _VP]),
    "dflash_add_rmsnorm_capture": (
        _I, [_VP, _VP, _VP, _I, _VP, _VP, _VP, _I64, _VP, _I, _I, ctypes.c_float, _VP]),
    "dflash_add_rmsnorm_splitk": (
        _I, [_VP, _VP, _I, _VP, _VP, _VP, _I, _I, ctypes.c_float, _VP]),
    "dflash_embed_rmsnorm": (_I, [_VP, _VP, _I, _VP, _VP, _VP, _I, _I, ctypes.c_float, _VP]),
    "dflash_gemm_bf16": (_I, [_VP, _I64, _VP, _I64, _VP, _I64, _I, _I, _I, _I, _I, _I, _VP]),
    "dflash_gemm_splits": (_I, [_I, _I]),
    "dflash_gemm_bf16_swiglu": (_I, [_VP, _I64, _VP, _I64, _VP, _I64, _I, _I, _I, _I, _VP]),
    "dflash_weight_tile_bytes": (_SZ, [_I, _I]),
    "dflash_weight_tile_bf16": (_I, [_VP, _I64, _VP, _I, _I, _VP]),
    "dflash_gemm_bf16_tiled": (
        _I, [_VP, _I64, _VP, _VP, _I64, _I, _I, _I, _I, _I, _I, _VP, _SZ, _VP]),
    "dflash_gemm_bf16_swiglu_tiled": (
        _I, [_VP, _I64, _VP, _VP, _I64, _I, _I, _I, _I, _VP, _SZ, _VP]),
    "dflash_gemm_tail_workspace_bytes": (_SZ, []),
    "dflash_gemm_bf16_tiled_residual_norm": (
        _I, [_VP, _I64, _VP, _I, _I, _I, _VP, _VP, _VP, _I64, _VP, _VP]),
    "dflash_gemm_bf16_tiled_normed": (
        _I, [_VP, _I64, _VP, _VP, _I, ctypes.c_float, _VP, _VP, _VP, _I64, _I, _I, _I, _I, _I, _I,
             _VP, _SZ, _VP]),
    "dflash_gemm_bf16_swiglu_tiled_normed": (
        _I, [_VP, _I64, _VP, _VP, _I, ctypes.c_float, _VP, _VP, _VP, _I64, _I, _I, _I, _I, _VP,
             _SZ, _VP]),
    "dflash_gemm_bf16_tiled_prefill": (_I, [_VP, _I64, _VP, _VP, _I64, _I, _I, _I, _VP]),
    "dflash_gemm_bf16_swiglu_tiled_prefill": (_I, [_VP, _I64, _VP, _VP, _I64, _I, _I, _I, _VP]),
    "dflash_gemm_bf16_tiled_prefill_splitk": (_I, [_VP, _I64, _VP, _VP, _I, _I, _I, _I, _VP]),
    "dflash_gemm_bf16_tiled_prefill_rows": (
        _I, [_VP, _I64, _VP, _I, _I, _VP, _I64, _VP, _I, _I, _I, _I, _I, _VP]),
    "dflash_splitk_reduce": (_I, [_VP, _I, _I, _I, _VP, _I64, _VP]),
    "dflash_splitk_swiglu_reduce": (_I, [_VP, _I, _I, _I, _VP, _I64, _VP]),
    "dflash_swiglu": (_I, [_VP, _VP, _I, _I, _VP]),
    "dflash_attn_prep": (
        _I,
        [_VP, _I64, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I, _I,
         ctypes.c_float, ctypes.c_float, _VP],
    ),
    "dflash_attn_verify_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "dflash_attn_verify": (
        _I,
        [_VP, _VP, _VP, _VP, _VP, _I64, _VP, _I, _I, _I, _I, _I, _I, _I, ctypes.c_float, _VP,
         _SZ, _VP],
    ),
    "dflash_attn_prefill": (
        _I,
        [_VP, _VP, _VP, _VP, _VP, _I64, _VP, _I, _I, _I, _I, _I, ctypes.c_float, _VP],
    ),
    "dflash_commit_accept": (_I, [_VP, _VP, _VP, _I, _I, _VP]),
    "dflash_greedy_accept_workspace_bytes": (_SZ, [_I, _I, _I]),
    "dflash_greedy_accept_noalloc_max_bytes": (_SZ, []),
    "dflash_greedy_accept_noalloc": (
        _I, [_VP, _I, _I64, _I64, _VP, _I64, _I, _VP, _VP, _VP, _I, _I, _I, _VP]),
    "dflash_greedy_accept": (
        _I,
        [_VP, _I, _I64, _I64, _VP, _I64, _I, _VP, _VP, _VP, _I, _I, _I, _VP, _SZ, _VP],
    ),
    "dflash_gdn_prologue": (
        _I,
        [_VP, _I64, _I64, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
         _I, _I, _I, _I, _I, _I, _I, ctypes.c_float, _VP],
    ),
    "dflash_gdn_prologue_scan_rollback": (
        _I,
        [_VP, _I64, _I64, _VP, _VP, _VP, _VP, _VP, _VP, _VP,  # prologue inputs
         _VP, _VP, _VP, _I, _I, _VP, _VP, _VP,  # state, selection, outputs
         _I, _I, _I, _I, _I, _I, _I, ctypes.c_float, _VP],
    ),
    "dflash_gdn_gated_rmsnorm": (
        _I, [_VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, ctypes.c_float, _VP]),
    "dflash_lm_head_accept_workspace_bytes": (_SZ, [_I, _I, _I]),
    "dflash_lm_head_greedy_accept": (
        _I,
        [_VP, _I64, _VP, _I64, _I, _I, _VP, _I64, _I, _VP, _VP, _VP, _I, _I, _VP, _SZ, _VP],
    ),
    "dflash_lm_head_greedy_accept_tiled": (
        _I,
        [_VP, _I64, _VP, _I, _I, _VP, _I64, _I, _VP, _VP, _VP, _I, _I, _VP, _SZ, _VP],
    ),
    "dflash_greedy_accept_conv_rollback": (
        _I,
        [_VP, _I, _I64, _I64, _VP, _I64, _I, _VP, _VP, _VP, _I, _I, _I, _VP, _SZ,  # accept
         _VP, _VP, _VP, _I, _VP, _I, _I, _I, _I64, _I64, _I64, _I, _VP],  # conv rollback
    ),
    "dflash_accept_keys_conv_rollback": (
        _I,
        [_VP, _I64, _I, _VP, _VP, _VP, _I, _I, _I, _VP, _SZ,
         _VP, _VP, _VP, _I, _VP, _I, _I, _I, _I64, _I64, _I64, _I, _VP],
    ),
    "dflash_tape_select": (_I, [_VP, _VP, _VP, _VP, _I, _I, _I, _I64, _I64, _VP]),
    "dflash_conv_rollback": (
        _I,
        [_VP, _VP, _VP, _VP, _I, _I, _I, _I, _I64, _I64, _I64, _I, _VP],
    ),
}
ABI_VERSION = 4

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class DFlashError(RuntimeError):
    """A libdflash entry point returned a non-zero status."""

    def __init__(self, fn: str, code: int, text: str):
        super().__init__(f"{fn} failed with code {code}: {text}")
        self.fn = fn
        self.code = code


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m dflash_mlx._build` "
                "(or __graft_entry__.build()) first"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        got = lib.dflash_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH.name} has ABI {got}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


def check(fn: str, code: int) -> None:
    if code != 0:
        text = load().dflash_strerror(code).decode(errors="replace")
        raise DFlashError(fn, code, text)


def call(fn: str, *args) -> None:
    check(fn, getattr(load(), fn)(*args))


def ptr(t: "torch.Tensor | None") -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: "torch.device") -> int:
    """hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr_array(tensors) -> ctypes.Array:
    """Host array of device pointers, for the multi-layer entry points."""
    arr = (ctypes.c_void_p * len(tensors))()
    for i, t in enumerate(tensors):
        arr[i] = t.data_ptr()
    return arr


def dtype_tag(dt: "torch.dtype") -> int:
    if dt == torch.float32:
        return DFLASH_DTYPE_F32
    if dt == torch.bfloat16:
        return DFLASH_DTYPE_BF16
    if dt == torch.float16:
        return DFLASH_DTYPE_F16
    raise TypeError(f"unsupported dtype {dt}")
