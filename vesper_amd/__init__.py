"""vesper_amd: MI355X-native quantized MoE expert arithmetic behind Vesper's Python interface.

The compute path is libmxmoe.so (hand-written HIP for gfx950, C ABI in
include/mxmoe.h), loaded with ctypes by `vesper_amd._lib`. Modules mirror the
reference's interface for this path:

  expert.ExpertExecutor / ResidentExpert      src/vesper/expert.py
  shared.ResidentSharedExpert                 src/vesper/shared.py
  moe.participation / MoEAccumulator          src/vesper/moe.py
  router.RouterProbe / GateProjection         src/vesper/router.py, src/vesper/gate.py
  connected.ConnectedMoE / ConnectedConfig    src/vesper/connected.py (ConnectedLayer: same call, resident)
  tiered.CacheConfig / TieredExpertRuntime    src/vesper/tiered.py
  cache.TieredCache                           src/vesper/cache.py
  store.NativeStore / build_store             src/vesper/storage.py
  fixtures.load_{gate,router,shared}_fixture  src/vesper/gate.py, router.py, shared.py
  disk.DirectReader, resources.MemoryBudget   src/vesper/disk.py, src/vesper/resources.py
  integrity.DeviceIntegrity                   src/vesper/integrity.py
  conformance.compare + format hooks          src/vesper/conformance.py
  layer.ExpertBank / MoELayer                 batched decode entry (T <= 16 tokens per call)
"""

from .config import BASELINE, REFERENCE, MoEConfig

__all__ = ["MoEConfig", "BASELINE", "REFERENCE"]
