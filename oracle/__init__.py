"""CPU oracle for the ctmr conv3d / group-norm hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline).  The product path (``mlx-generate-ctmr_amd``) never imports it and
has no CPU fallback.

Modules:
  reference_math  float64 NumPy restatements of the reference's operator math
                  (conv3d stride 1/2 and 1x1, nearest-2x parity fold, trilinear
                  2x, group norm + SiLU, average pooling), each citing the
                  reference file:line it follows.

Pinning (how each function is checked, see ``tests/test_oracle.py``):
  conv3d          golden ``source_fp32.npz:output.conv`` (Torch CPU recording),
                  brute-force loops on tiny inputs, torch.nn.functional.conv3d
                  in float64, 1x1 == matmul, stride 2 == subsampled stride 1.
  fold_upsample   exact identity with conv of the materialized nearest-2x
                  upsampling (float64), golden-free but closed-form.
  upsample_*      golden ``output.trilinear``; F.interpolate (trilinear,
                  align_corners=False / nearest) in float64.
  group_norm      goldens ``output.norm`` and ``output.vae_norm``;
                  F.group_norm in float64; invariance to per-group shifts.
  silu            golden ``output.silu``; closed form at special points.
  avg_pool        F.avg_pool3d in float64.
No function is left "parity unpinned".
"""
