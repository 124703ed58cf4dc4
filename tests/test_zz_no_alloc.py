"""r2s_rasterize_fwd_noalloc_*: the rasterizer forward with its split partial
tiles in the library's static device array instead of a caller's workspace.

Called through the C ABI on two scenes in a row, the second smaller (fewer
tiles, fewer splits, so the array still holds the first call's partial tiles
beyond what the second writes), each with heavy tiles split across blocks;
the image must equal r2s_rasterize_fwd_*'s with a workspace bit for bit (the
same kernels, the same split count, the same summation order).
"""

import math

import pytest
import torch

from r2splat import geometry, scenes
from r2splat.cuda import _backend, _ops
from r2splat.cuda import _wrapper as W

pytestmark = pytest.mark.gpu
DEV = "cuda"
TS = 16


def _inputs(n, det, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    raw = scenes.random_gaussians(n, g, log_scale_mu=-2.5, log_scale_sigma=0.3, extent=0.5)
    cov, _, op = W.prepare_gaussians(raw.quats.to(DEV), raw.raw_scales.to(DEV),
                                     raw.raw_opacities.to(DEV), 5e-4, 1.0)
    vm, Ks = geometry.cone_beam_views([math.radians(20.0 + seed)], det)
    t = lambda a: a.to(device=DEV, dtype=dtype).contiguous()  # noqa: E731
    m2, _, radii, con, mu, wt = W.project_gaussians_fwd(t(raw.means), t(cov), t(op), t(vm),
                                                        t(Ks), det, det, 1e-8, 3.0)
    nt = -(-det // TS)
    lists = _ops.bin_tiles_2d(m2, radii, TS, nt, nt)
    off = W.isect_offset_encode(lists.isect_ids, 1, nt, nt)
    return dict(m2=m2, con=con, op=wt, mu=mu, off=off, fl=lists.flatten_ids, det=det, nt=nt,
                n=lists.flatten_ids.numel(), N=m2.shape[1])


def _render(lib, d, noalloc, dtype):
    P, sfx = _ops._ptr, "f32" if dtype == torch.float32 else "f64"
    det, nt = d["det"], d["nt"]
    image = torch.full((1, det, det), float("nan"), dtype=dtype, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    args = (P(d["m2"]), P(d["con"]), P(d["op"]), P(d["mu"]), P(d["off"]), P(d["fl"]), d["n"], 1,
            d["N"], det, det, TS, nt, nt, P(image))
    if noalloc:
        rc = getattr(lib, f"r2s_rasterize_fwd_noalloc_{sfx}")(*args, stream)
    else:
        ws_bytes = lib.r2s_rasterize_workspace_bytes(nt * nt, d["n"], TS, image.element_size())
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
        rc = getattr(lib, f"r2s_rasterize_fwd_{sfx}")(*args, P(ws), ws_bytes, stream)
    assert rc == 0, lib.r2s_last_error()
    torch.cuda.synchronize()
    return image


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_noalloc_forward_equals_workspace_forward_on_two_calls(dtype):
    lib = _backend.library()
    scenes_ = [_inputs(80_000, 128, 1, dtype), _inputs(30_000, 96, 2, dtype)]
    used = []
    for d in scenes_:
        need = lib.r2s_rasterize_workspace_bytes(d["nt"] ** 2, d["n"], TS,
                                                 torch.tensor([], dtype=dtype).element_size())
        print(f"{dtype} det {d['det']}: {d['n']} records, partial tiles {need} bytes", flush=True)
        assert 0 < need <= (32 << 20)  # heavy tiles are split, the array holds them
        used.append(need)
    assert used[1] < used[0]
    for d in scenes_:  # the first call, then the smaller second one
        got = _render(lib, d, True, dtype)
        want = _render(lib, d, False, dtype)
        assert torch.isfinite(got).all() and float(got.abs().sum()) > 0
        assert torch.equal(got, want)
