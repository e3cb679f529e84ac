"""CPU oracle for the Gaussian-splatting rasterizer -- TEST INFRASTRUCTURE ONLY.

A restatement, in PyTorch (CPU) and numpy, of the reference's pure-Torch
rasterizer (src/torch_rasterizer.py, src/gaussian.py:6-79) and of the integer
binning semantics of src/cuda/kernel.cu:784-914 and
scripts/check_cuda_gradients.py:57-193.  Each function cites the reference
lines it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker / the timed CPU baseline.  The product
(3dgs_from_scratch_amd/cuda_rasterizer) never calls it: there is no CPU
fallback.

Modules:
  preprocess  projection to the image plane and spherical harmonics
  binning     tile rectangles, 64-bit keys, stable sort, tile ranges (numpy)
  blend       per-tile vectorised compositing (the Torch rasterizer's loop) and
              a brute-force per-pixel loop
  render      the full render pipeline (src/torch_rasterizer.py:9-290)

Pinning (how each part is checked independently of its own formulas) is listed
in tests/test_oracle.py's module docstring.
"""
