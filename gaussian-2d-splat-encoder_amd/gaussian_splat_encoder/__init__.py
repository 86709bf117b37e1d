"""MI355X-native tile-binned Gaussian-splat renderer (gfx950 HIP kernels behind a C-ABI).

Public entry points (the reference's render API):
  render_hip.render_alpha_octave, render_alpha_full_triton, render_alpha_multires, PairBudgetExceeded
  render.render_alpha_full, render_alpha_subsampled, _pixels
  params.activate_scale, SCALE_EPS, assemble_gaussian_params
"""
