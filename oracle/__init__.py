"""CPU oracle for the tile-binned splat renderer. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only
as the checker. The product path (the HIP library and its Python host) never imports, links or calls
anything here.

Contents and what pins each part (a function with no independent check says "parity unpinned"):

* binning.py (numpy, fp32 op by op)  -- render_triton.py:351-409 `_build_tiles`.
  Pinned by: the independent C restatement in oracle.c (loop form + counting sort), an exact-rational
  model of the fp32 rect arithmetic (tests/test_oracle_binning.py), brute-force rect/tile enumeration on
  tiny inputs, CSR invariants, and boundary cases (splats exactly on tile edges, off-canvas clamping,
  fused-multiply-add traps).
* oracle.c (C, float64 geometry over the fp32 pair list) -- render_triton.py:423-517 (cull forward) and
  602-720 (cull backward, the reference's analytic per-pair gradient formulas), 364-409 (binning).
  Pinned by: agreement with render_ref.py's autograd gradients, and through it central differences.
* render_ref.py (torch float64 on CPU) -- render.py:34-110 (exact materialised path), render_triton.py:
  423-517 (cull fields/composite, alpha and odds), 864-980 (multires/octave glue), 1431-1457 (odds).
  Pinned by: closed forms (single splat, opacity -> 0, the 1-1e-4 clamp, theta=None == theta=0),
  central finite differences of the autograd gradients, the cull->exact convergence as the cutoff grows,
  and the reference's own identities (fields == composite, octave(max_octaves=0) == cull).
"""
