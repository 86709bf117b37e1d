"""Import-path compatibility for callers written against the reference (`from .render_triton import ...`,
efficient_encoder.py:27-28 and examples/encode_and_render.py:16). Re-exports the HIP renderer's entry
points under that module path; there is no Triton anywhere in this package."""

from .render_hip import (PairBudgetExceeded, _build_tiles, _octave_of, _upsample_field,  # noqa: F401
                         render_alpha_full_triton, render_alpha_multires, render_alpha_octave)
