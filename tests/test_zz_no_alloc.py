"""GPU test of the entry point that allocates nothing (g2v_cosine_loss_forward_noalloc), through the
C ABI: on two calls in a row, the second with a smaller grid, its loss and valid-voxel count equal
those of g2v_cosine_loss_forward (the workspace entry point, same kernels) bit for bit, and the
oracle's within 1e-4.  Also: the library's scratch is the only device memory it uses (the caching
allocator's count does not move across the calls), and an oversized count is rejected."""
import ctypes
import sys

import numpy as np
import pytest
import torch

from oracle import g2v_oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _inputs(shape, C, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    label = torch.randint(0, 3, shape, generator=g).to(torch.float32)
    mask = torch.rand(shape, generator=g) < 0.8
    p = torch.randn(*shape, C, generator=g)
    t = torch.randn(*shape, C, generator=g)
    return label, mask, p.to(dtype), t.to(dtype)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def test_noalloc_forward_matches_workspace_forward_twice():
    from CudaGaussianVoxelizer import _lib
    lib = _lib.load()
    dev = torch.device("cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    fdt = {torch.float32: _lib.G2V_DTYPE_F32, torch.bfloat16: _lib.G2V_DTYPE_BF16}
    cases = [((40, 40, 16), 96, 1, torch.float32), ((12, 10, 8), 24, 2, torch.float32),
             ((30, 20, 8), 64, 3, torch.bfloat16), ((5, 4, 3), 8, 4, torch.bfloat16)]
    for shape, C, seed, dtype in cases:   # each second call of a type is the smaller one
        say(f"[noalloc] grid {shape} C={C} {dtype}")
        label, mask, p, t = (x.to(dev) for x in _inputs(shape, C, seed, dtype))
        V = label.numel()
        out = torch.empty(4, dtype=torch.float32, device=dev)     # loss, count (as int) x 2 calls
        cnt = torch.empty(2, dtype=torch.int32, device=dev)
        ws = torch.empty(lib.g2v_cosine_loss_workspace(V, C), dtype=torch.uint8, device=dev)
        _lib.check(lib.g2v_cosine_loss_forward(V, C, _ptr(label), _ptr(mask), _ptr(p), _ptr(t), fdt[dtype],
                                               _ptr(out[0:1]), _ptr(cnt[0:1]), None, _ptr(ws), ws.numel(), stream),
                   "g2v_cosine_loss_forward")
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated(dev)
        _lib.check(lib.g2v_cosine_loss_forward_noalloc(V, C, _ptr(label), _ptr(mask), _ptr(p), _ptr(t), fdt[dtype],
                                                       _ptr(out[1:2]), _ptr(cnt[1:2]), stream),
                   "g2v_cosine_loss_forward_noalloc")
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated(dev) == before
        assert out[0].item() == out[1].item() and cnt[0].item() == cnt[1].item(), (out, cnt)
        ref_loss, ref_cnt = O.cosine_loss_f64(label.cpu().numpy(), mask.cpu().numpy(),
                                              p.float().cpu().numpy(), t.float().cpu().numpy())
        assert cnt[1].item() == ref_cnt
        assert abs(out[1].item() - ref_loss) <= 1e-4 * max(abs(ref_loss), 1e-30)


def test_noalloc_forward_rejects_oversized_count():
    from CudaGaussianVoxelizer import _lib
    lib = _lib.load()
    one = ctypes.c_void_p(16)
    rc = lib.g2v_cosine_loss_forward_noalloc(1 << 31, 8, one, one, one, one, 0, one, one, None)
    assert rc == 3 and b"int32" in lib.g2v_last_error()
