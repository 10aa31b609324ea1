"""Writes tests/golden/mmdet_debug_inputs.npz from the reference's recorded training batch.

The reference ships debug_gaussian_voxelizer_output.pth (read by its test/test_data_from_mmdetection.py):
the Gaussians of one ShelfGaussian batch, means (1,6,300,3) float32, opacities (1,6,300,1) float32,
covariances (1,6,300,3,3) float16, voxelized on the 200x200x16 grid of 0.4 m voxels over
[-40,-40,-1,40,40,5.4].  Its recorded densities predate the current kernels (reference
test/README.md) and are not kept: the fixture holds the inputs only, flattened to 1,800
Gaussians, with the covariances kept in float16 so that the values are exactly the recorded ones.

Run once in a checkout next to the reference (the loader executes nothing from the file):
    python tests/golden/make_mmdet_fixture.py /path/to/reference/debug_gaussian_voxelizer_output.pth
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def main(path):
    d = torch.load(path, map_location="cpu", weights_only=True)
    means = d["means3d"].detach().reshape(-1, 3).to(torch.float32).numpy()
    opac = d["opacities"].detach().reshape(-1).to(torch.float32).numpy()
    cov = d["covariances"].detach().reshape(-1, 9).numpy()
    assert cov.dtype == np.float16 and means.shape[0] == opac.shape[0] == cov.shape[0]
    np.savez_compressed(os.path.join(HERE, "mmdet_debug_inputs.npz"), means3D=means, opacity=opac,
                        covariances_f16=cov, voxel_size=np.array([0.4, 0.4, 0.4], np.float32),
                        voxel_range=np.array([-40.0, -40.0, -1.0, 40.0, 40.0, 5.4], np.float32))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/debug_gaussian_voxelizer_output.pth")
