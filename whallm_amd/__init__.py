"""whallm_amd -- MI355X (gfx950) decode-time token selection for Whallm.

Hand-written HIP kernels (libwh_sample.so, C ABI in include/wh_sample.h)
for Whallm's penalty processors, temperature, top-k / top-p / min-p filters,
categorical draw and DSpark/MTP speculative verification, with drop-in
mirrors of the reference's Python call signatures:

    whallm_amd.sample_utils  -- mlx_lm make_sampler / make_logits_processors / apply_*
    whallm_amd.dspark        -- sampling_logprobs / _sample / _verify / DraftResult
    whallm_amd.sampling      -- batched fused entry points (sample, verify_fused, ...)
"""
from . import _lib  # noqa: F401

__all__ = ["sampling", "sample_utils", "dspark"]
__version__ = "0.1.0"
