"""GPU checks of the measurement workloads in the runtime: the streaming read kernel that gives the HBM
read rate the weight-streaming kernels are compared with must read every word of its range exactly once.
"""

import numpy as np
import pytest

from vesper_amd import _lib

pytestmark = pytest.mark.gpu

WORKGROUPS = 4096
STEP = 4096


def test_read_kernel_reads_every_word_of_its_range(gpu_ctx):
    """Workgroup g owns the contiguous range g; wave w reads its 4 KB steps w, w + 4, ...: the XOR each
    wave writes equals the XOR of exactly those words (a skipped or doubled step changes it)."""
    rng = np.random.default_rng(4096)
    nbytes = WORKGROUPS * STEP * 14                        # 14 steps per workgroup: the loop and its remainder
    words = rng.integers(0, 2 ** 32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    src = gpu_ctx.upload(words)
    out = gpu_ctx.empty((WORKGROUPS * 4,), np.uint32)
    try:
        with pytest.raises(ValueError):
            gpu_ctx.lib.read_kernel(gpu_ctx._h(), _lib.vp(src), nbytes - STEP, _lib.vp(out), None)
        gpu_ctx.lib.read_kernel(gpu_ctx._h(), _lib.vp(src), nbytes, _lib.vp(out), None)
        gpu_ctx.sync()
        got = out.download().reshape(WORKGROUPS, 4)
        steps = words.reshape(WORKGROUPS, nbytes // WORKGROUPS // STEP, STEP // 4)
        for w in range(4):
            want = np.bitwise_xor.reduce(steps[:, w::4, :].reshape(WORKGROUPS, -1), axis=1)
            np.testing.assert_array_equal(got[:, w], want, err_msg=f"wave {w}")
    finally:
        src.free()
        out.free()
