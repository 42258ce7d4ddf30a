"""The C-ABI library loads, exports every symbol include/litemoe_amd.h
declares, and its host-side checks work without a GPU (no kernel launches)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from litemoe_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "litemoe_amd.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|const char \*)\s*(lm_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    handle = _lib.load()
    names = declared()
    assert len(names) >= 15
    assert sorted(_lib.EXPORTED) == names
    for name in names:
        assert hasattr(handle, name), name


def test_version_and_status_strings():
    handle = _lib.load()
    assert b"gfx950" in handle.lm_version()
    assert handle.lm_status_string(0) == b"ok"
    assert handle.lm_status_string(4) == b"workspace too small"


def test_workspace_queries():
    # tokens 64, top-8, hidden 1536, inter 512, 40 experts (the 3B decode shape)
    size = _lib.size_query("lm_fused_experts_workspace_size", 64, 8, 1536, 512, 40)
    routes = 64 * 8
    assert size == 256 + 4 * routes + 2 * routes * 512 + 2 * routes * 1536
    assert _lib.size_query("lm_flash_decode_workspace_size", 64, 24, 64, 1) == 0
    n = 64 * 24 * 5
    assert _lib.size_query("lm_flash_decode_workspace_size", 64, 24, 64, 5) == n * 256 + 2 * n * 4
    # fused head: one 8-byte argmax word per row and slice of 8 vocabulary tiles (4 waves x 2 tiles);
    # 49155 rows are 3073 tiles of 16, i.e. 385 slices
    assert _lib.size_query("lm_head_greedy_workspace_size", 64, 49155, 1536) == 64 * 385 * 8
    assert _lib.size_query("lm_head_greedy_workspace_size", 128, 49155, 1536) == 128 * 385 * 8
    assert _lib.size_query("lm_head_greedy_workspace_size", 16, 1000, 512) == 16 * 8 * 8


# Non-null dummy pointers: every case returns before any launch, so nothing
# is dereferenced (the checks run on the host only).
_P = 16


@pytest.mark.parametrize("call,expected", [
    (lambda h: h.lm_rmsnorm(None, None, None, -1, 16, C.c_float(1e-6), None), 1),
    (lambda h: h.lm_flash_decode(None, 0, 0, None, None, None, 1, 4, 2, 8, 128, C.c_float(1.0), 8, 1, None, None,
                                 0, None), 2),
    (lambda h: h.lm_moe_align(None, 4, 0, 600, None, None, None, None), 2),
    (lambda h: h.lm_fused_experts(None, None, None, None, None, None, 4, 1000, 512, 8, 2, 0, None, None, 0, None), 2),
    (lambda h: h.lm_moe_finish(None, None, None, None, None, None, 1, 8, 9, 0, 1, None, 0, None), 1),
    (lambda h: h.lm_router(None, None, 2, 1536, 300, 8, 1, None, None, None, None), 2),
    # fragment-order entry points: more than 128 rows, K not a multiple of 32
    (lambda h: h.lm_linear_splitk_frag(None, None, 129, 512, 1024, 2, None, None), 2),
    (lambda h: h.lm_linear_splitk_frag(None, None, 4, 512, 1000, 2, None, None), 1),
    (lambda h: h.lm_flash_decode_qkv_frag(None, 3, None, 16, None, None, None, None, None, None, 200, 24, 8,
                                          1024, 64, C.c_float(1.0), 1024, 1, None, None, 0, None), 2),
    # dense projection: K not a multiple of 64, strides below K, misaligned operands, null pointers
    (lambda h: h.lm_linear(_P, 96, _P, 96, 4, 32, 96, _P, 32, None), 2),
    (lambda h: h.lm_linear(_P, 64, _P, 128, 4, 32, 128, _P, 32, None), 1),
    (lambda h: h.lm_linear(_P + 2, 128, _P, 128, 4, 32, 128, _P, 32, None), 1),
    (lambda h: h.lm_linear(None, 128, _P, 128, 4, 32, 128, _P, 32, None), 1),
    (lambda h: h.lm_linear(None, 128, None, 128, 0, 32, 128, None, 32, None), 0),
])
def test_invalid_arguments_rejected_on_host(call, expected):
    assert call(_lib.load()) == expected


@pytest.mark.parametrize("name,call,expected", [
    ("topk > 8", lambda h: h.lm_fused_experts(_P, _P, _P, _P, _P, None, 4, 1024, 512, 16, 9, 0, _P, _P, 1 << 30,
                                                None), 1),
    ("block_rows % 16", lambda h: h.lm_fused_experts(_P, _P, _P, _P, _P, None, 4, 1024, 512, 16, 2, 8, _P, _P,
                                                       1 << 30, None), 1),
    ("experts > 511", lambda h: h.lm_fused_experts(_P, _P, _P, _P, _P, None, 4, 1024, 512, 600, 2, 0, _P, _P,
                                                     1 << 30, None), 1),
    ("topk > experts", lambda h: h.lm_moe_routes(_P, _P, _P, _P, 4, 1024, 512, 2, 4, 0, _P, _P, 1 << 30, None), 1),
    ("null workspace", lambda h: h.lm_moe_routes(_P, _P, _P, _P, 4, 1024, 512, 8, 2, 0, _P, None, 1 << 30, None),
     1),
    ("workspace short", lambda h: h.lm_fused_experts(_P, _P, _P, _P, _P, None, 4, 1024, 512, 8, 2, 0, _P, _P, 100,
                                                       None), 4),
    ("routes workspace short", lambda h: h.lm_moe_routes(_P, _P, _P, _P, 64, 1536, 512, 40, 8, 0, _P, _P, 4096,
                                                           None), 4),
    ("hidden 1000", lambda h: h.lm_moe_routes(_P, _P, _P, _P, 4, 1000, 512, 8, 2, 0, _P, _P, 1 << 30, None), 2),
    ("scan path > 256 tokens", lambda h: h.lm_moe_gate_up(_P, _P, None, None, _P, 300 * 2, 2, 1024, 512, 8, 0,
                                                             _P, None), 2),
    ("splitk rows 129", lambda h: h.lm_linear_splitk(_P, 1536, _P, 129, 2560, 1536, 3, _P, None), 2),
    ("splitk bad slices", lambda h: h.lm_linear_splitk(_P, 1536, _P, 64, 2560, 1536, 5, _P, None), 2),
    ("flash workspace short", lambda h: h.lm_flash_decode(_P, 64 * 24, 64, _P, _P, _P, 64, 24, 8, 2048, 64,
                                                            C.c_float(0.125), 2048, 4, _P, _P, 16, None), 4),
    ("finish topk 9", lambda h: h.lm_moe_finish(_P, _P, None, _P, None, _P, 1, 8, 9, 0, 1, None, 0, None), 1),
    ("head rows 129", lambda h: h.lm_head_greedy(_P, 1536, _P, 129, 49155, 1536, C.c_float(8.0), None, 0, _P, _P,
                                                   _P, _P, _P, _P, _P, None, 0, 1, None, 0, None, _P, 1 << 30, None),
     2),
    ("head hidden 1000", lambda h: h.lm_head_greedy(_P, 1000, _P, 64, 49155, 1000, C.c_float(8.0), None, 0, _P,
                                                      _P, _P, _P, _P, _P, _P, None, 0, 1, None, 0, None, _P, 1 << 30,
                                                      None), 2),
    ("head workspace short", lambda h: h.lm_head_greedy(_P, 1536, _P, 64, 49155, 1536, C.c_float(8.0), None, 0,
                                                          _P, _P, _P, _P, _P, _P, _P, None, 0, 1, None, 0, None, _P,
                                                          64 * 8, None), 4),
    ("head z misaligned", lambda h: h.lm_head_greedy(_P + 2, 1536, _P, 64, 49155, 1536, C.c_float(8.0), None, 0,
                                                       _P, _P, _P, _P, _P, _P, _P, None, 0, 1, None, 0, None, _P,
                                                       1 << 30, None), 1),
    ("head scaling 0", lambda h: h.lm_head_greedy(_P, 1536, _P, 64, 49155, 1536, C.c_float(0.0), None, 0, _P, _P,
                                                    _P, _P, _P, _P, _P, None, 0, 1, None, 0, None, _P, 1 << 30, None),
     1),
    ("pack hidden 1000", lambda h: h.lm_expert_pack(_P, _P, 8, 1000, 512, _P + 4096, _P + 8192, None), 2),
    ("pack aliasing", lambda h: h.lm_expert_pack(_P, _P + 4096, 8, 1024, 512, _P, _P + 8192, None), 1),
    ("pack misaligned", lambda h: h.lm_expert_pack(_P + 2, _P + 4096, 8, 1024, 512, _P + 8192, _P + 16384, None),
     1),
    ("prefill out misaligned", lambda h: h.lm_prefill_attention(_P, 2560, 64, _P, 2560, 64, _P, 2560, 64, _P, 2,
                                                                  128, 64, 24, 8, 64, C.c_float(0.125), 1, _P + 2,
                                                                  None), 1),
    ("prefill q stride 2564", lambda h: h.lm_prefill_attention(_P, 2564, 64, _P, 2560, 64, _P, 2560, 64, _P, 2,
                                                                 128, 64, 24, 8, 64, C.c_float(0.125), 1, _P, None),
     1),
    ("routes packed workspace short", lambda h: h.lm_moe_routes_packed(_P, _P, _P, _P, 64, 1536, 512, 40, 8, 0, _P,
                                                                         _P, 4096, None), 4),
    # QKV projection with the RoPE/KV epilogue: K not a multiple of 64, misaligned output, one cache pointer
    ("rope_kv K 96", lambda h: h.lm_linear_rope_kv(_P, 96, _P, 4, 24, 8, 96, _P, 2560, _P, None, None, _P, 64,
                                                     _P, _P, 64, 1, None), 2),
    ("rope_kv out misaligned", lambda h: h.lm_linear_rope_kv(_P, 128, _P, 4, 24, 8, 128, _P + 4, 2560, _P, None,
                                                               None, _P, 64, _P, _P, 64, 1, None), 1),
    ("rope_kv one cache", lambda h: h.lm_linear_rope_kv(_P, 128, _P, 4, 24, 8, 128, _P, 2560, _P, None, None, _P,
                                                          64, _P, None, 64, 1, None), 1),
    ("rope_kv ldo short", lambda h: h.lm_linear_rope_kv(_P, 128, _P, 4, 24, 8, 128, _P, 2048, _P, None, None, _P,
                                                          64, _P, _P, 64, 1, None), 1),
    ("ok: rope_kv zero rows", lambda h: h.lm_linear_rope_kv(None, 128, None, 0, 24, 8, 128, None, 2560, None, None,
                                                              None, None, 64, None, None, 64, 1, None), 0),
    # chained decode: residual and out both given, topk 9, outside the scan path, short workspace
    ("combine residual and out", lambda h: h.lm_moe_routes_combine(_P, _P, _P, _P, _P, 64, 1536, 512, 40, 8, _P,
                                                                     C.c_float(0.2), _P, _P, _P, 1 << 30, None), 1),
    ("combine topk 9", lambda h: h.lm_moe_routes_combine(_P, _P, _P, _P, _P, 64, 1536, 512, 40, 9, None,
                                                           C.c_float(0.0), None, _P, _P, 1 << 30, None), 1),
    ("combine 300 tokens", lambda h: h.lm_moe_routes_combine_packed(_P, _P, _P, _P, _P, 300, 1536, 512, 40, 8,
                                                                      None, C.c_float(0.0), None, _P, _P, 1 << 30,
                                                                      None), 2),
    ("combine workspace short", lambda h: h.lm_moe_routes_combine(_P, _P, _P, _P, _P, 64, 1536, 512, 40, 8, None,
                                                                    C.c_float(0.0), None, _P, _P, 64, None), 4),
    ("splitk_rmsnorm K 1536+64", lambda h: h.lm_linear_splitk_rmsnorm(_P, _P, _P, C.c_float(1e-6), _P, 64, 2560,
                                                                        1600, 3, _P, None), 2),
    ("splitk_rmsnorm null sumsq", lambda h: h.lm_linear_splitk_rmsnorm(_P, None, _P, C.c_float(1e-6), _P, 64,
                                                                         2560, 1536, 3, _P, None), 1),
    ("ok: zero tokens", lambda h: h.lm_fused_experts(_P, _P, _P, _P, _P, None, 0, 1024, 512, 8, 2, 0, _P, _P, 0,
                                                       None), 0),
])
def test_status_codes_before_launch(name, call, expected):
    """Each entry point reports a bad call with its status code (LM_EINVAL 1,
    LM_EUNSUPPORTED 2, LM_EWORKSPACE 4) before it launches anything, and
    lm_status_string names it."""
    handle = _lib.load()
    assert call(handle) == expected, name
    assert handle.lm_status_string(expected) != b"unknown status"


def test_single_hip_runtime_in_process():
    import torch  # noqa: F401  (loads torch's HIP runtime)
    _lib.load()
    _lib._check_single_runtime()
