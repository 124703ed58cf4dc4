"""CPU oracle for the r2splat Gaussian backend -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithms of the BT-3DGS ``r2splat``
CUDA operators (``r2splat/cuda/csrc/*.cu`` in the reference tree).  Each
function cites the reference ``file:line`` it follows.  It is the checker for
the HIP kernels, never part of the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and the shipped ``r2splat`` package never does.

Modules
-------
``ops``      numpy restatements of the element-wise operators (parameter
             transform, cone-beam projection, conics/mu, volume mapping),
             written in the reference kernels' operation order so that fp32
             results are reproducible bit-for-bit where no transcendental
             function is involved.
``binning``  integer tile binning (count, emit, stable sort, offsets), 2D and
             3D, plus the densify/prune index compaction.
``native``   ctypes bindings of ``oracle/c/r2s_oracle.c``: the rasterizer and
             voxelizer (forward and both backward modes), over OpenMP
             threads with results independent of the thread count.
``compose``  the ``r2splat.ops`` forward/backward composition on top of the
             above (explicit.py / direct.py restated).
``dense``    the reference's dense PyTorch formulation (every Gaussian at
             every pixel / voxel, torch autograd backward): the CPU
             baseline's workload, checked against the modules above.

Seeded synthetic inputs come from ``r2splat.scenes`` / ``r2splat.geometry``
(host-side generators, no device code).  How each function is pinned (the
reference's known-answer tests, closed forms, autograd, finite differences,
brute force, invariants) is listed in ``tests/test_oracle_*.py``; every
function has at least one such check, so none is "parity unpinned".
Fixtures produced by this oracle are committed under ``tests/golden/``.
"""
