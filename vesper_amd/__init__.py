"""vesper_amd: MI355X-native quantized MoE expert arithmetic behind Vesper's Python interface.

The compute path is libmxmoe.so (hand-written HIP for gfx950, C ABI in
include/mxmoe.h), loaded with ctypes by `vesper_amd._lib`. Modules mirror the
reference's interface for this path:

  expert.ExpertExecutor / ResidentExpert      src/vesper/expert.py
  shared.ResidentSharedExpert                 src/vesper/shared.py
  moe.participation / MoEAccumulator          src/vesper/moe.py
  router.RouterProbe / GateProjection         src/vesper/router.py, src/vesper/gate.py
  connected.ConnectedMoE                      src/vesper/connected.py
  conformance.compare + format hooks          src/vesper/conformance.py
  layer.ExpertBank / MoELayer                 batched decode entry (T <= 16 tokens per call)
"""

from .config import BASELINE, REFERENCE, MoEConfig

__all__ = ["MoEConfig", "BASELINE", "REFERENCE"]
