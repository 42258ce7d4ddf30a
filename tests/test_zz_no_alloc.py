"""lm_fused_experts_noalloc against lm_fused_experts, through the C ABI.

The no-allocation entry point carves its workspace from a static device
array instead of a caller buffer; its results must be bitwise those of the
workspace entry point on the same inputs. Two calls in a row, the second
with a smaller input (the array keeps the first call's contents), and a
call beyond the array's size, which must be refused before any launch.
"""
import pytest
import torch

from litemoe_amd import _lib
from litemoe_amd.synth import normal_bf16
from oracle import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
LM_ETOOLARGE = 5


def _inputs(m, h, i, e, k, seed):
    x = normal_bf16((m, h), 1.0, seed)
    w1 = normal_bf16((e, 2 * i, h), 0.02, seed + 1)
    w2 = normal_bf16((e, h, i), 0.02, seed + 2)
    wr = normal_bf16((e, h), 0.02, seed + 3)
    weights, ids = ops.route(torch.nn.functional.linear(x, wr), k)
    return [t.to(DEV).contiguous() for t in (x, w1, w2, weights.float(), ids.int())]


def _with_workspace(x, w1, w2, weights, ids):
    m, h = x.shape
    e, two_i, _ = w1.shape
    k = ids.shape[1]
    nbytes = _lib.size_query("lm_fused_experts_workspace_size", m, k, h, two_i // 2, e)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    out = torch.empty_like(x)
    _lib.call("lm_fused_experts", x.data_ptr(), w1.data_ptr(), w2.data_ptr(), weights.data_ptr(), ids.data_ptr(),
              None, m, h, two_i // 2, e, k, 0, out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream(x.device))
    return out


def _no_alloc(x, w1, w2, weights, ids):
    m, h = x.shape
    e, two_i, _ = w1.shape
    out = torch.empty_like(x)
    _lib.call("lm_fused_experts_noalloc", x.data_ptr(), w1.data_ptr(), w2.data_ptr(), weights.data_ptr(),
              ids.data_ptr(), None, m, h, two_i // 2, e, ids.shape[1], 0, out.data_ptr(),
              _lib.stream(x.device))
    return out


@torch.inference_mode()
def test_no_alloc_equals_workspace_entry_point_twice_then_smaller():
    # first the 3B decode shape (scan path), then a smaller call of a
    # different geometry: the array still holds the first call's act and y
    for m, h, i, e, k, seed in ((64, 1536, 512, 40, 8, 11), (5, 1024, 512, 32, 8, 12)):
        args = _inputs(m, h, i, e, k, seed)
        got = _no_alloc(*args)
        expected = _with_workspace(*args)
        torch.cuda.synchronize()
        assert torch.equal(got, expected), (m, h, i, e, k)
        assert got.abs().sum() > 0


@torch.inference_mode()
def test_no_alloc_block_path_and_limit():
    # 300 tokens: the aligned-block path (offsets, sorted routes, act, y in the array)
    args = _inputs(300, 1024, 512, 32, 8, 13)
    assert torch.equal(_no_alloc(*args), _with_workspace(*args))
    # 4096 tokens x top-8 at hidden 1536 needs ~134 MB of workspace: refused
    # before any launch (the pointers are never read)
    handle = _lib.load()
    status = handle.lm_fused_experts_noalloc(16, 16, 16, 16, 16, None, 4096, 1536, 512, 40, 8, 0, 16, None)
    assert status == LM_ETOOLARGE
    assert b"scratch" in handle.lm_status_string(status)
