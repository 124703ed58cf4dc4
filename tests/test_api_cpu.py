"""Import and error contract of the r2splat package on a machine without a GPU."""

import os
import subprocess
import sys
import textwrap

import pytest
import torch


PKG = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "bt-3dgs_amd")


def test_import_does_not_touch_the_gpu():
    # Mirrors tests/test_release_imports.py:9-34 of the reference.
    code = textwrap.dedent("""
        import sys
        sys.path[:0] = [%r]
        import r2splat, r2splat.ops, r2splat.ops.direct, r2splat.ops.explicit
        import r2splat.cuda._wrapper
        from r2splat.cuda import _backend
        assert _backend._lazy_C._load_attempted is False
        print("ok")
    """ % PKG)
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip().endswith("ok")


def test_public_names_match_reference():
    import r2splat
    import r2splat.ops as ops
    from r2splat.cuda import _wrapper
    from r2splat.ops import direct, explicit

    for name in ("ExplicitGaussianState", "InferenceGaussianState", "MappingVoxelizationResult",
                 "ProjectionRasterizationResult", "inference_rasterize", "inference_voxelize",
                 "prepare_inference_gaussians"):
        assert hasattr(ops, name)
    for name in ("explicit_backward", "explicit_rasterize", "explicit_voxelize",
                 "prepare_explicit_gaussians"):
        assert hasattr(explicit, name)
    for name in ("isect_tiles", "parameter_transform_fwd", "parameter_transform_bwd",
                 "isect_offset_encode", "isect_tiles_3d", "isect_offset_encode_3d",
                 "conics_mu_fwd", "conics_mu_bwd", "world_to_image_projection_fwd",
                 "world_to_image_projection_bwd", "world_to_volume_mapping_fwd",
                 "world_to_volume_mapping_bwd", "rasterize_to_pixels_fwd",
                 "rasterize_to_pixels_bwd", "rasterize_to_pixels_bwd_per_gaussian",
                 "voxelize_to_voxels_fwd", "voxelize_to_voxels_bwd",
                 "voxelize_to_voxels_bwd_per_gaussian", "is_cuda_extension_available"):
        assert callable(getattr(_wrapper, name)), name
    assert r2splat.__version__
    fields = [f for f in direct.InferenceGaussianState.__dataclass_fields__]
    assert fields == ["covars", "max_scales", "opacities"]
    with pytest.raises(Exception):
        direct.InferenceGaussianState(torch.zeros(1), torch.zeros(1), torch.zeros(1)).covars = 1


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU failure mode")
def test_no_cpu_fallback():
    from r2splat.cuda import _wrapper
    from r2splat.ops import direct, explicit

    assert _wrapper.is_cuda_extension_available() is False
    with pytest.raises(RuntimeError, match="unavailable"):
        _wrapper.conics_mu_fwd(torch.zeros(1, 1, 6), 1e-8)
    q, s, o = torch.zeros(2, 4), torch.zeros(2, 3), torch.zeros(2)
    with pytest.raises(RuntimeError, match="require CUDA tensors"):
        direct.prepare_inference_gaussians(q, s, o, scale_min=5e-4, scale_max=1.0)
    with pytest.raises(ValueError, match="backward_mode"):
        explicit.prepare_explicit_gaussians(q, s, o, scale_min=5e-4, scale_max=1.0,
                                            backward_mode="x")
