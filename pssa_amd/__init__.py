"""MI355X (gfx950) PSSA inference forward path.

Host-side mirror of the reference's backend surface (Sparticle62ops/pssa):
`HipDevice` is the `GpuDispatch` peer (src/backend.rs:1025-1446) and
`PSSALayer` carries `forward_inference` / `prefill_inference`
(src/pssa.rs:2387-2442).  All compute runs in libpssa_hip.so (hand-written HIP
for gfx950, C ABI in include/pssa_hip.h).
"""
from .weights import BlockWeights, ModelWeights, PSSAConfig, bf16_round  # noqa: F401
from .checkpoint import load as load_checkpoint  # noqa: F401
from .device import HipDevice, PSSALayer, Sequence  # noqa: F401
