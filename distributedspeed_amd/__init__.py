"""distributedspeed_amd -- MI355X-native ZeRO optimizer step.

The hot path of DistributedSpeed's ZeROOptimizer.step
(Src/zero/optimizer.py:212-274) -- unscale, inf/NaN detection, grad norm,
clipping, AdamW, the 16-bit cast and the dynamic loss scaler -- as gfx950
HIP kernels behind a C ABI (include/dsx.h, libdsx.so).
"""
__version__ = "0.1.0"
