"""ctypes binding of the gfx950 C-ABI library ``_native/liblitemoe_amd.so``.

The library is the only compute path of this package: there is no CPU or
PyTorch fallback. :func:`lib` raises if the library is missing, and every
wrapper below raises if a call returns a nonzero status. This mirrors the
reference's own ctypes adapter (litemoe/ops.py:84-138), which binds a
vendor library and turns a nonzero status into ``RuntimeError``.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_native" / "liblitemoe_amd.so"

_v, _i64, _i32, _f32 = C.c_void_p, C.c_int64, C.c_int, C.c_float

# name -> argument types (all functions return int status unless listed in _RESTYPE).
_SIGNATURES = {
    "lm_version": [],
    "lm_status_string": [_i32],
    "lm_rmsnorm": [_v, _v, _v, _i64, _i64, _f32, _v],
    "lm_add_rmsnorm": [_v, _v, _f32, _v, _v, _i64, _i64, _f32, _v],
    "lm_kv_write": [_v, _i64, _i64, _i64, _v, _i64, _i64, _i64, _v, _v, _v, _v, _v,
                    _i64, _i64, _i64, _i64, _i64, _i64, _v],
    "lm_rope_kv_write": [_v, _i64, _i64, _v, _i64, _i64, _v, _i64, _i64, _v, _i64, _v, _v, _v,
                         _v, _v, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _v],
    "lm_flash_decode_workspace_size": [_i64, _i64, _i64, _i64, C.POINTER(C.c_int64)],
    "lm_flash_decode": [_v, _i64, _i64, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _f32, _i64,
                        _i64, _v, _v, _i64, _v],
    "lm_prefill_attention": [_v, _i64, _i64, _v, _i64, _i64, _v, _i64, _i64, _v, _i64, _i64,
                             _i64, _i64, _i64, _i64, _f32, _i32, _v, _v],
    "lm_router": [_v, _v, _i64, _i64, _i64, _i64, _i32, _v, _v, _v, _v],
    "lm_topk_softmax": [_v, _i64, _i64, _i64, _i32, _v, _v, _v],
    "lm_moe_align": [_v, _i64, _i64, _i64, _v, _v, _v, _v],
    "lm_fused_experts_workspace_size": [_i64, _i64, _i64, _i64, _i64, C.POINTER(C.c_int64)],
    "lm_fused_experts": [_v, _v, _v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _i64, _v, _v,
                         _i64, _v],
    "lm_fused_experts_noalloc": [_v, _v, _v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _i64, _v, _v],
    "lm_moe_gate_up": [_v, _v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _i64, _v, _v],
    "lm_moe_down": [_v, _v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _v, _v],
    "lm_moe_finish": [_v, _v, _v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _v, _i64, _v],
    "lm_add_rmsnorm_router": [_v, _v, _f32, _v, _f32, _v, _v, _i64, _i64, _i64, _i64, _i32, _v, _v, _v, _v],
    "lm_moe_routes_workspace_size": [_i64, _i64, _i64, _i64, _i64, C.POINTER(C.c_int64)],
    "lm_moe_routes": [_v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _i64, _v, _v, _i64, _v],
    "lm_moe_gate_up_packed": [_v, _v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _i64, _v, _v],
    "lm_moe_down_packed": [_v, _v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _v, _v],
    "lm_moe_routes_packed": [_v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _i64, _v, _v, _i64, _v],
    "lm_expert_pack": [_v, _v, _i64, _i64, _i64, _v, _v, _v],
    "lm_moe_routes_combine_workspace_size": [_i64, _i64, _i64, _i64, _i64, C.POINTER(C.c_int64)],
    "lm_moe_routes_combine": [_v, _v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _v, _f32, _v, _v, _v, _i64,
                              _v],
    "lm_moe_routes_combine_packed": [_v, _v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _v, _f32, _v, _v, _v,
                                     _i64, _v],
    "lm_fused_experts_packed": [_v, _v, _v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64, _i64, _v, _v,
                                _i64, _v],
    "lm_moe_finish_add_rmsnorm": [_v, _v, _v, _v, _v, _f32, _v, _f32, _v, _i64, _i64, _i64, _v],
    "lm_linear_splitk": [_v, _i64, _v, _i64, _i64, _i64, _i64, _v, _v],
    "lm_linear_splitk_frag": [_v, _v, _i64, _i64, _i64, _i64, _v, _v],
    "lm_linear_splitk_reduce": [_v, _i64, _i64, _i64, _v, _i64, _v],
    "lm_linear_splitk_rmsnorm": [_v, _v, _v, _f32, _v, _i64, _i64, _i64, _i64, _v, _v],
    "lm_linear": [_v, _i64, _v, _i64, _i64, _i64, _i64, _v, _i64, _v],
    "lm_linear_rope_kv": [_v, _i64, _v, _i64, _i64, _i64, _i64, _v, _i64, _v, _v, _v, _v, _i64, _v, _v, _i64,
                          _i64, _v],
    "lm_flash_decode_qkv": [_v, _i64, _v, _i64, _v, _v, _v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64,
                            _f32, _i64, _i64, _v, _v, _i64, _v],
    "lm_flash_decode_qkv_frag": [_v, _i64, _v, _i64, _v, _v, _v, _v, _v, _v, _i64, _i64, _i64, _i64, _i64,
                                 _f32, _i64, _i64, _v, _v, _i64, _v],
    "lm_add_rmsnorm_router_splitk": [_v, _v, _i64, _f32, _v, _f32, _v, _v, _i64, _i64, _i64, _i64,
                                     _i32, _v, _v, _v, _v],
    "lm_decode_prologue": [_v, _v, _v, _v, _f32, _v, _f32, _v, _v, _v, _v, _v, _v, _v, _i64, _i64, _i64,
                           _v],
    "lm_greedy_epilogue_workspace_size": [_i64, _i64, C.POINTER(C.c_int64)],
    "lm_greedy_epilogue": [_v, _i64, _f32, _i64, _i64, _v, _v, _v, _v, _v, _v, _v, _v, _i64, _i32,
                           _v, _i64, _v, _v, _i64, _v],
    "lm_host_device_pointer": [_v, C.POINTER(C.c_void_p)],
    "lm_head_pack_size": [_i64, _i64, C.POINTER(C.c_int64)],
    "lm_head_pack": [_v, _i64, _i64, _v, _v],
    "lm_head_greedy_workspace_size": [_i64, _i64, _i64, C.POINTER(C.c_int64)],
    "lm_head_greedy": [_v, _i64, _v, _i64, _i64, _i64, _f32, _v, _i64, _v, _v, _v, _v, _v, _v, _v, _v,
                       _i64, _i32, _v, _i64, _v, _v, _i64, _v],
}
_RESTYPE = {"lm_version": C.c_char_p, "lm_status_string": C.c_char_p}

EXPORTED = tuple(_SIGNATURES)

_LIB = None


class NativeError(RuntimeError):
    """A C-ABI call returned a nonzero status."""


def load(path: Path | str = LIB_PATH) -> C.CDLL:
    """Open the library and declare every exported signature (no GPU needed)."""
    if not Path(path).exists():
        raise RuntimeError(
            f"litemoe_amd native library not found at {path}; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` or `make -C litemoe_amd/csrc`")
    handle = C.CDLL(str(path))
    for name, args in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, C.c_int)
    return handle


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = load()
        _check_single_runtime()
    return _LIB


def _check_single_runtime():
    """The library must share torch's HIP runtime (one copy in the process)."""
    try:
        maps = Path("/proc/self/maps").read_text().splitlines()
    except OSError:
        return
    copies = {line.split()[-1] for line in maps if "libamdhip64" in line}
    if len(copies) > 1:
        raise RuntimeError(f"Two HIP runtimes are loaded: {sorted(copies)}")


def call(name: str, *args) -> None:
    status = getattr(lib(), name)(*args)
    if status:
        message = lib().lm_status_string(status).decode()
        raise NativeError(f"{name} failed with status {status} ({message})")


def size_query(name: str, *args) -> int:
    out = C.c_int64(0)
    call(name, *args, C.byref(out))
    return int(out.value)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_cuda(*tensors: torch.Tensor, what: str = "tensors") -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError(f"{what} must be on a ROCm device; this path has no CPU fallback")


def version() -> str:
    return lib().lm_version().decode()


if os.environ.get("LITEMOE_AMD_EAGER_LOAD") == "1":  # pragma: no cover
    lib()
