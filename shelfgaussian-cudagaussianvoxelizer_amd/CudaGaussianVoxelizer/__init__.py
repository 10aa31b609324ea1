"""MI355X (gfx950) Gaussian-to-Voxel splatting with the reference's Python API.

Mirrors CudaGaussianVoxelizer/__init__.py of lunarlab-gatech/ShelfGaussian-CudaGaussianVoxelizer
(lines 1-96): ``PyCudaGaussianVoxelizer(voxel_size, voxel_range)`` returns
``(density, grid_feats, stats)``; ``stats`` is a CPU float32 tensor ``[fwd_sec, bwd_sec]``,
the backward time being filled in when ``.backward()`` runs.  The kernels live in
libg2v_hip.so (C ABI in include/g2v.h), reached through the ``_C`` module.
"""
import torch
import torch.nn as nn

from . import _C
from ._C import gaussian_voxelizer_forward, gaussian_voxelizer_backward
from ._C import CudaFeatsCosinelossForward, CudaFeatsCosinelossBackward, gaussian_voxelizer_forward_batched

__all__ = ["PyCudaGaussianVoxelizer", "PyCudaFeatsCosineLoss", "PyCudaGaussianVoxelizerCosineLoss", "_C",
           "gaussian_voxelizer_forward", "gaussian_voxelizer_backward", "gaussian_voxelizer_forward_batched",
           "CudaFeatsCosinelossForward", "CudaFeatsCosinelossBackward", "covariance_from_scale_rotation"]


def _wants_backward(ctx, need_backward):
    """Whether the forward should keep and prepare what the backward reuses.  Inside
    Function.forward grad mode is always off, so the caller's grad mode arrives as need_backward
    (the module passes it); without it, whether any input requires grad decides."""
    if need_backward is not None:
        return bool(need_backward)
    return any(ctx.needs_input_grad)


def _grad_possible(*tensors):
    """A backward can follow this forward: grad mode is on and an input requires grad."""
    return torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors)


class _CudaGaussianVoxelizeFunction(torch.autograd.Function):
    """Autograd wrapper (reference CudaGaussianVoxelizer/__init__.py:10-47)."""

    @staticmethod
    def forward(ctx, means3D, opacity, covariances, voxel_size, voxel_range, features, need_backward=None):
        # with features the backward reuses the forward's Tile->Gaussian CSR (kept beside the
        # reference's saved tensors) instead of re-sorting the G->T pairs, and its workspace is
        # prepared behind the forward; without features only the grid values and the gradient
        # buffers are kept; all of it only when a backward can follow (need_backward, or when not
        # given, whether an input requires grad), so that an inference forward allocates and
        # launches nothing for a backward that never runs
        keep = _wants_backward(ctx, need_backward)
        (density, cov_inv, valid_voxel_lb, valid_voxel_ub, num_valid_voxel, grid_feats, g2t_offsets,
         g2t_tile_ids, fwd_sec), t2g = _C._forward(means3D, opacity, covariances, voxel_size,
                                                   voxel_range, features, keep_t2g=keep)
        stats = torch.zeros(2, dtype=torch.float32, device="cpu")
        stats[0] = fwd_sec
        ctx.save_for_backward(means3D, opacity, voxel_size, voxel_range, cov_inv, valid_voxel_lb,
                              valid_voxel_ub, num_valid_voxel, g2t_offsets, g2t_tile_ids, density,
                              grid_feats, features, stats)
        ctx.t2g = t2g
        ctx.mark_non_differentiable(stats)
        ctx.opacity_shape = opacity.shape
        ctx.cov_shape = covariances.shape
        return density, grid_feats, stats

    @staticmethod
    def backward(ctx, grad_density_output, grad_feats_output, grad_stats):
        (means32, op32, voxsz32, voxrg32, cov_inv, valid_voxel_lb, valid_voxel_ub, num_valid_voxel,
         g2t_offsets, g2t_tile_ids, density, grid_feats, features, stats) = ctx.saved_tensors
        gout32 = grad_density_output.to(torch.float32).contiguous()
        grad_feats_output = grad_feats_output.to(grid_feats.dtype).contiguous()   # the features' type
        means32 = means32.detach().contiguous()
        op32 = op32.detach().reshape(-1).contiguous()
        feats = None if features is None else features.detach().contiguous()
        grad_means3D, grad_cov, grad_opacity, grad_feats, bwd_sec = _C._backward(
            gout32, grad_feats_output, means32, op32, cov_inv, voxsz32, voxrg32, valid_voxel_lb,
            valid_voxel_ub, num_valid_voxel, g2t_offsets, g2t_tile_ids, density, grid_feats, feats,
            t2g=ctx.t2g)
        ctx.t2g = None
        stats[1] = bwd_sec
        # gradients take the shapes of the inputs ((N,) or (N,1) opacity, (N,9) or (N,3,3) cov)
        grad_opacity = grad_opacity.reshape(ctx.opacity_shape)
        grad_cov = grad_cov.reshape(ctx.cov_shape)
        return (grad_means3D, grad_opacity, grad_cov, None, None,
                grad_feats if features is not None else None, None)


class _CudaFeatsCosinelossFunction(torch.autograd.Function):
    """Autograd wrapper of the cosine loss (reference CudaGaussianVoxelizer/__init__.py:49-67):
    the gradient flows to d_grid_feats only."""

    @staticmethod
    def forward(ctx, voxel_label, occ_gt_mask_camera, d_grid_feats, pseudo_dino_gt):
        loss, num_valid_voxel, fwd_sec = CudaFeatsCosinelossForward(voxel_label, occ_gt_mask_camera,
                                                                    d_grid_feats, pseudo_dino_gt)
        stats = torch.zeros(2, dtype=torch.float32, device="cpu")
        stats[0] = fwd_sec
        ctx.save_for_backward(voxel_label, occ_gt_mask_camera, d_grid_feats, pseudo_dino_gt, stats)
        ctx.num_valid_voxel = num_valid_voxel
        return loss, stats

    @staticmethod
    def backward(ctx, grad_output, grad_stats):
        voxel_label, occ_gt_mask_camera, d_grid_feats, pseudo_dino_gt, stats = ctx.saved_tensors
        gout32 = grad_output.to(torch.float32).contiguous()
        grad_predict, bwd_sec = CudaFeatsCosinelossBackward(gout32, voxel_label, occ_gt_mask_camera,
                                                            d_grid_feats, pseudo_dino_gt, ctx.num_valid_voxel)
        stats[1] = bwd_sec
        return None, None, grad_predict, None


def _fusable(grid_feats, pseudo_dino_gt):
    """The fused cosine gradient applies: float32 rows of a multiple of 4 channels, 16-byte aligned."""
    return (grid_feats.dtype == torch.float32 and pseudo_dino_gt.dtype == torch.float32
            and grid_feats.shape[-1] > 0 and grid_feats.shape[-1] % 4 == 0
            and grid_feats.data_ptr() % 16 == 0 and pseudo_dino_gt.data_ptr() % 16 == 0)


class _CudaGaussianVoxelizeCosineLossFunction(torch.autograd.Function):
    """The voxelizer (reference CudaGaussianVoxelizer/__init__.py:10-47) followed by the feature
    cosine loss on its grid_feats (:49-67), with the loss's gradient fused into the voxelizer's
    backward: the (X,Y,Z,C) gradient of grid_feats that the reference writes between the two
    backwards is formed per voxel inside the feature-gradient kernels (_C.gaussian_voxelizer_
    backward_cosine).  float32 inputs with C % 4 == 0 take the fused kernels; other feature types
    chain the two backwards.  grid_feats keeps its gradient path: when another use of it sends a
    gradient back, that gradient is added to the loss's (materialised, as the chained modules do)
    and the voxelizer's backward reads the sum."""

    @staticmethod
    def forward(ctx, means3D, opacity, covariances, voxel_size, voxel_range, features, voxel_label,
                occ_gt_mask_camera, pseudo_dino_gt, need_backward=None):
        if features is None or features.shape[-1] == 0:
            raise RuntimeError("the cosine loss needs features")
        keep = _wants_backward(ctx, need_backward)
        (density, cov_inv, valid_voxel_lb, valid_voxel_ub, num_valid_voxel, grid_feats, g2t_offsets,
         g2t_tile_ids, fwd_sec), t2g = _C._forward(means3D, opacity, covariances, voxel_size,
                                                   voxel_range, features, keep_t2g=keep)
        fused = keep and _fusable(grid_feats, pseudo_dino_gt)
        loss, count, cos_sec, coef = _C._cosine_forward(voxel_label, occ_gt_mask_camera, grid_feats,
                                                        pseudo_dino_gt, fused)
        stats = torch.zeros(2, dtype=torch.float32, device="cpu")
        stats[0] = fwd_sec + cos_sec
        ctx.save_for_backward(means3D, opacity, voxel_size, voxel_range, cov_inv, valid_voxel_lb,
                              valid_voxel_ub, num_valid_voxel, g2t_offsets, g2t_tile_ids, density,
                              grid_feats, features, voxel_label, occ_gt_mask_camera, pseudo_dino_gt, coef,
                              stats)
        ctx.t2g = t2g
        ctx.count = count
        ctx.fused = fused
        ctx.mark_non_differentiable(stats)
        # no zero-filled (X,Y,Z,C) gradient for grid_feats: unused outputs arrive as None
        ctx.set_materialize_grads(False)
        ctx.opacity_shape = opacity.shape
        ctx.cov_shape = covariances.shape
        return density, loss, grid_feats, stats

    @staticmethod
    def backward(ctx, grad_density_output, grad_loss, grad_grid_feats, grad_stats):
        (means32, op32, voxsz32, voxrg32, cov_inv, valid_voxel_lb, valid_voxel_ub, num_valid_voxel,
         g2t_offsets, g2t_tile_ids, density, grid_feats, features, voxel_label, occ_gt_mask_camera,
         pseudo_dino_gt, coef, stats) = ctx.saved_tensors
        gout32 = torch.zeros_like(density) if grad_density_output is None else \
            grad_density_output.to(torch.float32).contiguous()
        gl32 = torch.zeros(1, dtype=torch.float32, device=density.device) if grad_loss is None else \
            grad_loss.detach().to(torch.float32).reshape(1).contiguous()
        means32 = means32.detach().contiguous()
        op32 = op32.detach().reshape(-1).contiguous()
        feats = features.detach().contiguous()
        saved = (means32, op32, cov_inv, voxsz32, voxrg32, valid_voxel_lb, valid_voxel_ub, num_valid_voxel,
                 g2t_offsets, g2t_tile_ids, density, grid_feats, feats)
        if ctx.fused and grad_grid_feats is None:
            res = _C._backward(gout32, None, *saved, t2g=ctx.t2g,
                               cosine=(gl32, pseudo_dino_gt, coef, ctx.count))
            bwd_sec = res[4]
        else:   # chained: the loss's gradient of grid_feats (plus another use's), then the voxelizer's backward
            grad_grid, cos_sec = _C.CudaFeatsCosinelossBackward(gl32, voxel_label, occ_gt_mask_camera, grid_feats,
                                                                pseudo_dino_gt, ctx.count)
            if grad_grid_feats is not None:
                grad_grid = grad_grid + grad_grid_feats.to(grad_grid.dtype)
            res = _C._backward(gout32, grad_grid, *saved, t2g=ctx.t2g)
            bwd_sec = res[4] + cos_sec
        grad_means3D, grad_cov, grad_opacity, grad_feats, _ = res
        ctx.t2g = None
        stats[1] = bwd_sec
        return (grad_means3D, grad_opacity.reshape(ctx.opacity_shape), grad_cov.reshape(ctx.cov_shape), None,
                None, grad_feats, None, None, None, None)


class _CudaGaussianVoxelizeBatchedFunction(torch.autograd.Function):
    """Autograd wrapper of B scenes on one grid (means3D (B,N,3)), run as one problem of B N
    Gaussians (one launch per kernel for the batch, one host wait for its plan); returns density
    (B,X,Y,Z), grid_feats (B,X,Y,Z,C) and stats."""

    @staticmethod
    def forward(ctx, means3D, opacity, covariances, voxel_size, voxel_range, features, need_backward=None):
        scenes, density, grid_feats, batch = _C._forward_batched(means3D, opacity, covariances, voxel_size,
                                                                 voxel_range, features,
                                                                 keep_t2g=_wants_backward(ctx, need_backward))
        stats = torch.zeros(2, dtype=torch.float32, device="cpu")
        stats[0] = scenes[0][8] if scenes else 0.0
        ctx.batch = batch
        ctx.grid = (voxel_size, voxel_range)
        ctx.save_for_backward(means3D, opacity, covariances, features, stats)
        ctx.mark_non_differentiable(stats)
        ctx.shapes = (means3D.shape, opacity.shape, covariances.shape)
        return density, grid_feats, stats

    @staticmethod
    def backward(ctx, grad_density_output, grad_feats_output, grad_stats):
        means3D, opacity, covariances, features, stats = ctx.saved_tensors
        B, n = means3D.shape[0], means3D.shape[1]
        m32 = means3D.detach().contiguous()
        o32 = opacity.detach().reshape(B, n).contiguous()
        feats = None if features is None else features.detach().contiguous()
        batch = ctx.batch
        if batch is None:   # the forward kept nothing for a backward (need_backward=False): redo its plan
            batch = _C._forward_batched(m32, o32, covariances.detach(), *ctx.grid, feats, keep_t2g=True)[3]
        if B == 0:
            gm, gc, go = m32.new_zeros(0, n, 3), m32.new_zeros(0, n, 9), m32.new_zeros(0, n)
            gf = None if feats is None else feats.new_zeros(feats.shape)
            bwd_sec = 0.0
        else:
            gD = grad_density_output.to(torch.float32).contiguous()
            gF = grad_feats_output.to(torch.float32 if features is None else features.dtype).contiguous()
            gm, gc, go, gf, bwd_sec = _C._backward_batched(gD, gF, m32, o32, feats, batch)
        ctx.batch = None
        stats[1] = bwd_sec
        return (gm.reshape(ctx.shapes[0]), go.reshape(ctx.shapes[1]), gc.reshape(ctx.shapes[2]), None, None,
                gf if features is not None else None, None)


class _CovarianceFromScaleRotation(torch.autograd.Function):
    """Covariances from scales and rotations (reference test/gaussian_voxelizer.py:14-37), with
    the chain rule back to both."""

    @staticmethod
    def forward(ctx, scales, rotations):
        ctx.save_for_backward(scales, rotations)
        ctx.shapes = (scales.shape, rotations.shape)
        return _C.covariance_from_scale_rotation(scales, rotations)

    @staticmethod
    def backward(ctx, grad_cov):
        scales, rotations = ctx.saved_tensors
        gs, gq = _C.covariance_from_scale_rotation_backward(scales, rotations, grad_cov.to(torch.float32))
        return gs.reshape(ctx.shapes[0]), gq.reshape(ctx.shapes[1])


def covariance_from_scale_rotation(scales, rotations):
    """(N, 9) covariances (R diag(s)) (R diag(s))^T of scales (N, 3) and quaternions (N, 4, real
    part first; normalised here), differentiable in both (reference
    test/gaussian_voxelizer.py:30-37 get_covariance of quat_to_rotmat)."""
    return _CovarianceFromScaleRotation.apply(scales, rotations)


class PyCudaGaussianVoxelizer(nn.Module):
    """Splats Gaussians (and their features) into a dense voxel grid of 4x4x4 tiles.

    Reference CudaGaussianVoxelizer/__init__.py:69-82.
    """

    def __init__(self, voxel_size=[0.4, 0.4, 0.4], voxel_range=[-40, -40, -1, 40, 40, 5.4]):
        super().__init__()
        self.voxel_size = torch.tensor(voxel_size, dtype=torch.float32, device="cuda")
        self.voxel_range = torch.tensor(voxel_range, dtype=torch.float32, device="cuda")
        # host copies, so the forward never reads the device tensors back
        _C._host_values(self.voxel_size, 3, "voxel_size")
        _C._host_values(self.voxel_range, 6, "voxel_range")

    def forward(self, means3D, opacity, covariances=None, features=None, *, scales=None, rotations=None):
        """As the reference's forward; without covariances, they are built from ``scales`` (N, 3)
        and ``rotations`` (N, 4) (as ShelfGaussian's voxelizer does, reference
        test/gaussian_voxelizer.py:168-169) and the gradients flow to those two.  Covariances may
        be float16 or bfloat16 and features bfloat16 (grid_feats and the feature gradient then
        are bfloat16 too).  With means3D of
        shape (B, N, 3) (opacity (B, N[, 1]), covariances (B, N, 9), features (B, N, C)) the B
        scenes are voxelized in one call: density (B, X, Y, Z), grid_feats (B, X, Y, Z, C)."""
        if covariances is None:
            if scales is None or rotations is None:
                raise RuntimeError("give covariances, or scales and rotations")
            covariances = covariance_from_scale_rotation(scales, rotations)
        if covariances.dtype in (torch.float16, torch.bfloat16):
            # reduced-precision covariances (ShelfGaussian records them in float16): widened on the
            # device, the gradient flows back in their type
            covariances = covariances.float()
        need = _grad_possible(means3D, opacity, covariances, features)
        if means3D.dim() == 3:   # B scenes on this grid: (B,N,3) means, outputs gain a leading B
            return _CudaGaussianVoxelizeBatchedFunction.apply(means3D, opacity, covariances, self.voxel_size,
                                                              self.voxel_range, features, need)
        return _CudaGaussianVoxelizeFunction.apply(means3D, opacity, covariances, self.voxel_size,
                                                   self.voxel_range, features, need)


class PyCudaGaussianVoxelizerCosineLoss(PyCudaGaussianVoxelizer):
    """PyCudaGaussianVoxelizer followed by PyCudaFeatsCosineLoss on its grid_feats, as one op whose
    backward forms the loss's gradient of grid_feats inside the voxelizer's feature-gradient kernels
    instead of writing and re-reading it (2.6 GB at 200 x 200 x 16 x 1024 float32).

    ``forward(means3D, opacity, covariances, features, voxel_label, occ_gt_mask_camera,
    pseudo_dino_gt)`` returns ``(density, loss, grid_feats, stats)``: density and loss carry
    gradients (to means3D, opacity, covariances and features), grid_feats does not, stats is the CPU
    float32 tensor ``[fwd_sec, bwd_sec]`` of both ops together.  One scene (means3D (N, 3)).
    """

    def forward(self, means3D, opacity, covariances, features, voxel_label, occ_gt_mask_camera, pseudo_dino_gt):
        if means3D.dim() != 2:
            raise RuntimeError("PyCudaGaussianVoxelizerCosineLoss takes one scene: means3D (N, 3)")
        if covariances.dtype in (torch.float16, torch.bfloat16):
            covariances = covariances.float()
        need = _grad_possible(means3D, opacity, covariances, features)
        return _CudaGaussianVoxelizeCosineLossFunction.apply(means3D, opacity, covariances, self.voxel_size,
                                                             self.voxel_range, features, voxel_label,
                                                             occ_gt_mask_camera, pseudo_dino_gt, need)


class PyCudaFeatsCosineLoss(nn.Module):
    """Mean voxel-wise cosine loss between grid features and pseudo ground-truth features over the
    voxels that are visible (occ_gt_mask_camera) and labelled (voxel_label > 0).

    Reference CudaGaussianVoxelizer/__init__.py:84-96; returns ``(loss, stats)`` with ``stats`` the
    CPU float32 tensor ``[fwd_sec, bwd_sec]``.  voxel_size and voxel_range are kept as the
    reference keeps them (unused by the loss).
    """

    def __init__(self, voxel_size=[0.4, 0.4, 0.4], voxel_range=[-40, -40, -1, 40, 40, 5.4]):
        super().__init__()
        self.voxel_size = torch.tensor(voxel_size, dtype=torch.float32, device="cuda")
        self.voxel_range = torch.tensor(voxel_range, dtype=torch.float32, device="cuda")

    def forward(self, voxel_label, occ_gt_mask_camera, d_grid_feats, pseudo_dino_gt):
        return _CudaFeatsCosinelossFunction.apply(voxel_label, occ_gt_mask_camera, d_grid_feats, pseudo_dino_gt)
