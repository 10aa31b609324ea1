"""The C-ABI library loads and exports every symbol of include/g2v.h; host-only entry points
(grid geometry, workspace queries, argument checks) behave.  No GPU needed: nothing here
launches a kernel."""
import ctypes
import os
import re

import numpy as np
import pytest

from oracle import g2v_oracle as O
from tests import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _lib():
    from CudaGaussianVoxelizer import _lib
    return _lib


def test_header_symbols_exported():
    text = open(os.path.join(ROOT, "include", "g2v.h")).read()
    names = sorted(set(re.findall(r"\b(g2v_[a-z0-9_]+)\s*\(", text)))
    assert len(names) >= 10
    lib = ctypes.CDLL(_lib().LIB_PATH)
    for n in names:
        assert hasattr(lib, n), n
    # the Python binding declares exactly the header's entry points
    assert set(names) == set(_lib().SIGNATURES)


def test_abi_version():
    assert _lib().load().g2v_abi_version() == _lib().ABI_VERSION == 13


def test_loader_refuses_other_abi(monkeypatch):
    """A library whose ABI differs from the one SIGNATURES describes is refused at load time."""
    L = _lib()
    monkeypatch.setattr(L, "ABI_VERSION", L.ABI_VERSION + 1)
    monkeypatch.setattr(L, "_lib", None)
    with pytest.raises(ImportError, match="rebuild"):
        L.load()


@pytest.mark.parametrize("vs,vr", [
    ([0.4] * 3, W.RANGE_PAPER), ([0.4] * 3, W.RANGE_SMALL),
    ([0.3] * 3, [0, 0, 0, 0.9, 0.9, 0.9]), ([0.1] * 3, [-1.3, -1.3, -1.3, 1.3, 1.3, 1.3]),
    ([0.5, 0.25, 0.2], [-7.0, -3.0, -2.0, 7.0, 3.1, 2.0]),
])
def test_grid_dims_matches_oracle(vs, vr):
    from CudaGaussianVoxelizer import _C
    assert _C.grid_dims(vs, vr) == O.grid_dims(vs, vr)


def test_bad_grid_reports_error():
    L = _lib()
    lib = L.load()
    dims = (ctypes.c_int * 3)()
    rc = lib.g2v_grid_dims(L.floats([0.0, 0.4, 0.4]), L.floats(W.RANGE_PAPER), dims, dims)
    assert rc == 1
    assert b"grid axis 0" in lib.g2v_last_error()
    with pytest.raises(RuntimeError, match="invalid argument"):
        L.check(rc, "g2v_grid_dims")


def test_invalid_arguments_fail_before_any_launch():
    L = _lib()
    lib = L.load()
    vs, vr = L.floats([0.4] * 3), L.floats(W.RANGE_PAPER)
    M = ctypes.c_longlong(0)
    # negative N
    rc = lib.g2v_forward_plan(-1, None, None, vs, vr, None, None, None, None, None, None, 0,
                              ctypes.byref(M), None, 0, None, None)
    assert rc == 1 and b"n = -1" in lib.g2v_last_error()
    # too many pairs for the int32 CSR
    rc = lib.g2v_forward_splat(1, 0, None, None, None, 0, None, 0, vs, vr, None, None, None, None, 1 << 31,
                               None, None, None, None, None, None, None, 0, None)
    assert rc == 3
    # unknown feature type
    rc = lib.g2v_forward_splat(1, 0, None, None, None, 7, None, 0, vs, vr, None, None, None, None, 0,
                               None, None, None, None, None, None, None, 0, None)
    assert rc == 1 and b"feat_dtype" in lib.g2v_last_error()
    # missing workspace
    rc = lib.g2v_forward_splat(0, 0, None, None, None, 0, None, 0, vs, vr, None, None, None, None, 0, None,
                               ctypes.c_void_p(16), None, None, None, None, None, 0, None)
    assert rc == 1 and b"workspace" in lib.g2v_last_error()
    # features without their packed rows
    rc = lib.g2v_forward_splat(4, 8, None, None, ctypes.c_void_p(16), 0, None, 0, vs, vr, None, None, None, None, 0,
                               None, ctypes.c_void_p(16), ctypes.c_void_p(16), None, None, None, None, 0, None)
    assert rc == 1 and b"packed_features" in lib.g2v_last_error()
    # packed rows of too few bytes for (n, feat_dim): rejected before anything is queued
    need = lib.g2v_forward_packed_bytes(4, 8)
    rc = lib.g2v_forward_splat(4, 8, None, None, ctypes.c_void_p(16), 0, ctypes.c_void_p(16), need - 1, vs, vr, None,
                               None, None, None, 0, None, ctypes.c_void_p(16), ctypes.c_void_p(16), None, None, None,
                               None, 0, None)
    assert rc == 1 and b"packed features buffer too small" in lib.g2v_last_error()
    # packing: buffer size, type and pointers are checked before anything is queued
    need = lib.g2v_forward_packed_bytes(4, 8)   # 5 rows (a zero row last) of channels padded to 128
    assert need == 5 * 128 * 4 and lib.g2v_forward_packed_bytes(4, 0) == 0
    rc = lib.g2v_forward_pack_features(4, 8, ctypes.c_void_p(16), 0, ctypes.c_void_p(16), need - 1, None)
    assert rc == 1 and b"too small" in lib.g2v_last_error()
    rc = lib.g2v_forward_pack_features(4, 8, ctypes.c_void_p(16), 5, ctypes.c_void_p(16), need, None)
    assert rc == 1 and b"feat_dtype" in lib.g2v_last_error()
    rc = lib.g2v_forward_pack_features(4, 8, None, 0, ctypes.c_void_p(16), need, None)
    assert rc == 1 and b"null" in lib.g2v_last_error()
    assert lib.g2v_forward_pack_features(4, 0, None, 0, None, 0, None) == 0
    # features requested without tensors
    rc = lib.g2v_backward(4, 8, ctypes.c_void_p(16), None, ctypes.c_void_p(16), ctypes.c_void_p(16),
                          ctypes.c_void_p(16), vs, vr, ctypes.c_void_p(16), ctypes.c_void_p(16), None,
                          None, None, 0, 0, None, None, None, 0, ctypes.c_void_p(16), ctypes.c_void_p(16),
                          ctypes.c_void_p(16), None, None, None, None, None, None, 0, None)
    assert rc == 1 and b"feat_dim" in lib.g2v_last_error()


def test_backward_prepare_arguments_fail_before_any_launch():
    L = _lib()
    lib = L.load()
    vs, vr = L.floats([0.4] * 3), L.floats(W.RANGE_PAPER)
    one = ctypes.c_void_p(16)
    rc = lib.g2v_backward_prepare(-1, 8, vs, vr, one, one, one, 0, 0, 0, one, one, one, one, 1 << 20, None)
    assert rc == 1 and b"n = -1" in lib.g2v_last_error()
    # the forward's Tile->Gaussian CSR is required
    rc = lib.g2v_backward_prepare(10, 8, vs, vr, one, one, one, 0, 100, 10, None, None, one, one, 1 << 30, None)
    assert rc == 1 and b"Tile->Gaussian" in lib.g2v_last_error()
    rc = lib.g2v_backward_prepare(10, 8, vs, vr, one, one, one, 0, 100, 10, one, one, one, one, 16, None)
    assert rc == 1 and b"workspace" in lib.g2v_last_error()
    assert lib.g2v_backward_prepare(10, 0, vs, vr, None, None, None, 0, 0, 0, None, None, None, None, 0, None) == 0
    rc = lib.g2v_backward_prepared(4, 8, one, one, one, one, one, vs, vr, one, one, None, one, one, 10, 5,
                                   one, one, one, 0, one, one, one, one, None, None, None, one, one, 1 << 30, None)
    assert rc == 1 and b"Tile->Gaussian" in lib.g2v_last_error()


def test_cosine_invalid_arguments_fail_before_any_launch():
    L = _lib()
    lib = L.load()
    cnt = ctypes.c_int(0)
    one = ctypes.c_void_p(16)
    rc = lib.g2v_cosine_loss_forward(-1, 8, None, None, None, None, 0, one, one, None, None, 0, None)
    assert rc == 1 and b"num_voxels = -1" in lib.g2v_last_error()
    rc = lib.g2v_cosine_loss_forward(1 << 31, 8, one, one, one, one, 0, one, one, None, one, 1 << 20, None)
    assert rc == 3
    rc = lib.g2v_cosine_loss_forward(64, 8, one, one, one, one, 0, None, one, ctypes.byref(cnt), one, 1 << 20, None)
    assert rc == 1 and b"null" in lib.g2v_last_error()
    rc = lib.g2v_cosine_loss_forward(64, 8, one, one, one, one, 0, one, one, None, one, 16, None)
    assert rc == 1 and b"workspace" in lib.g2v_last_error()
    rc = lib.g2v_cosine_loss_forward(64, 8, one, one, one, one, 2, one, one, None, one, 1 << 20, None)
    assert rc == 1 and b"feat_dtype" in lib.g2v_last_error()
    rc = lib.g2v_cosine_loss_backward(64, 8, None, one, one, one, one, 0, 3, one, None)
    assert rc == 1 and b"null" in lib.g2v_last_error()
    rc = lib.g2v_cosine_loss_backward(64, 8, one, one, one, one, one, 7, 3, one, None)
    assert rc == 1 and b"feat_dtype" in lib.g2v_last_error()
    # nothing to do: no launch, success
    assert lib.g2v_cosine_loss_backward(0, 8, None, None, None, None, None, 0, 0, None, None) == 0
    assert lib.g2v_cosine_loss_workspace(640_000, 1024) > 0


def test_workspace_queries_grow_with_problem():
    L = _lib()
    lib = L.load()
    vs, vr = L.floats([0.4] * 3), L.floats(W.RANGE_PAPER)
    a = lib.g2v_forward_splat_workspace(1000, 0, 10_000, vs, vr)
    b = lib.g2v_forward_splat_workspace(1000, 0, 1_000_000, vs, vr)
    assert a >= 1000 * 64   # the density-only splat packs a 64-byte record per Gaussian
    f1 = lib.g2v_forward_splat_workspace(1000, 64, 10_000, vs, vr)
    assert 0 < f1 < lib.g2v_forward_splat_workspace(1000, 64, 1_000_000, vs, vr)
    assert 0 < a < b
    assert lib.g2v_backward_workspace(1000, 64, 10_000, 2000, vs, vr) > lib.g2v_backward_workspace(1000, 0, 10_000, 0, vs, vr)
    assert lib.g2v_backward_workspace(1000, 64, 10_000, 4000, vs, vr) > lib.g2v_backward_workspace(1000, 64, 10_000, 2000, vs, vr)
    assert lib.g2v_forward_plan_workspace(200_000) > lib.g2v_forward_plan_workspace(10)


def test_batch_arguments_and_workspaces():
    """The batch entry points check their sizes before any launch, and a batch of B scenes needs
    the workspaces of one problem of B n Gaussians on B T tiles."""
    L = _lib()
    lib = L.load()
    vs, vr = L.floats([0.4] * 3), L.floats(W.RANGE_PAPER)
    one = ctypes.c_void_p(16)
    assert lib.g2v_batch_plan_workspace(0, 300) == 0
    assert lib.g2v_batch_plan_workspace(1 << 16, 1 << 16) == 0   # B n beyond int32
    p1, p6 = lib.g2v_batch_plan_workspace(1, 300), lib.g2v_batch_plan_workspace(6, 300)
    assert 0 < p1 < p6
    s1 = lib.g2v_batch_forward_splat_workspace(1, 300, 64, 10_000, vs, vr)
    s6 = lib.g2v_batch_forward_splat_workspace(6, 300, 64, 10_000, vs, vr)
    # six scenes hold six tile-offset arrays and a sort key per pair
    assert s6 > s1 >= lib.g2v_forward_splat_workspace(300, 64, 10_000, vs, vr)
    assert (lib.g2v_batch_backward_workspace(6, 300, 64, 10_000, 2000, vs, vr) >
            lib.g2v_batch_backward_workspace(1, 300, 64, 10_000, 2000, vs, vr))
    # B x 10,000 tiles beyond int32 (B n still fits): no size, as the plan would refuse it
    B = 300_000
    assert lib.g2v_batch_plan_workspace(B, 1) > 0
    assert lib.g2v_batch_forward_splat_workspace(B, 1, 64, 10_000, vs, vr) == 0
    assert lib.g2v_batch_backward_workspace(B, 1, 64, 10_000, 2000, vs, vr) == 0
    cnt = (ctypes.c_longlong * 8)()
    rc = lib.g2v_batch_forward_plan(0, 300, one, one, vs, vr, one, one, one, one, one, one, 1 << 20, 1, cnt, None)
    assert rc == 1 and b"num_scenes = 0" in lib.g2v_last_error()
    rc = lib.g2v_batch_forward_plan(2, 300, one, one, vs, vr, one, one, one, one, one, one, 16, 1, cnt, None)
    assert rc == 1 and b"workspace" in lib.g2v_last_error()
    rc = lib.g2v_batch_forward_plan(2, 300, one, one, vs, vr, one, one, one, one, None, one, 1 << 20, 1, cnt, None)
    assert rc == 1 and b"null" in lib.g2v_last_error()
    # the plan workspace of one scene is too small for two; a prepared backward needs the batch's CSR
    rc = lib.g2v_batch_backward(2, 300, 8, one, one, one, one, one, vs, vr, one, one, 100, 10, one, one, one, 0, one,
                                one, one, one, None, None, None, one, p1, one, 1 << 30, 1, None)
    assert rc == 1 and b"batch plan workspace" in lib.g2v_last_error()
    rc = lib.g2v_batch_backward(2, 300, 8, one, one, one, one, one, vs, vr, one, one, 100, 10, one, one, one, 0, one,
                                one, one, one, None, None, None, one, p6, one, 1 << 30, 1, None)
    assert rc == 1 and b"Tile->Gaussian" in lib.g2v_last_error()
def test_product_path_does_not_reference_oracle():
    pkg = os.path.join(ROOT, "shelfgaussian-cudagaussianvoxelizer_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.replace("reference", ""), f


def test_float_quotient_of_small_integers_is_exact():
    """The density backward finds a lane's box digits as int((float)a / (float)b) for 0 <= a < 2^23,
    b >= 1 (csrc/g2v_backward.hip, small_quot): a correctly rounded float32 quotient of such integers,
    truncated, is floor(a / b).  Checked with IEEE float32 division on random pairs, pairs just below
    and at multiples of b, and the extremes of the range."""
    rng = np.random.default_rng(7)
    a = rng.integers(0, 1 << 23, 400_000, dtype=np.int64)
    b = rng.integers(1, 1 << 23, 400_000, dtype=np.int64)
    small_b = rng.integers(1, 4097, 400_000, dtype=np.int64)
    q = rng.integers(0, 2048, 400_000, dtype=np.int64)
    near = np.clip(q * small_b + rng.integers(-1, 2, 400_000), 0, (1 << 23) - 1)   # around multiples of b
    edges_a = np.array([0, 1, (1 << 23) - 1, (1 << 23) - 2, (1 << 22), (1 << 22) - 1], dtype=np.int64)
    edges_b = np.array([1, 2, 3, (1 << 23) - 1, (1 << 22) + 1, 4095], dtype=np.int64)
    cases = [(a, b), (near, small_b), (a % 64, small_b)] + [(edges_a, np.full_like(edges_a, e)) for e in edges_b]
    for aa, bb in cases:
        got = (aa.astype(np.float32) / bb.astype(np.float32)).astype(np.int64)
        assert np.array_equal(got, aa // bb)
