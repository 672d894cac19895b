import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


class DequantRef:
    """Reference weights of a Q4 linear: `exact` is float(q) * scale (the
    dequantisation every path but one keeps exactly), `fp16` the weight tile
    the tiled GEMM multiplies when its plan reads fp16_dequant=1: fp16(q * s)
    with fp32 scales rounded to fp16 first (AEXQ_EPI_EXACT_DEQUANT off)."""

    def __init__(self, exact, fp16=None):
        self.exact = exact
        self.fp16 = exact if fp16 is None else fp16

    def for_plan(self, plan: str):
        return self.fp16 if "fp16_dequant=1" in plan else self.exact


def q4_reference(orc, words, scales, n, k, group, code, scale_f16):
    import numpy as np
    odt = orc.SCALE_F16 if scale_f16 else orc.SCALE_F32
    exact = orc.dequant_q4(words, scales, n, k, group, nibble_code=code, scale_dtype=odt)
    s16 = np.asarray(scales).astype(np.float16)
    w16 = orc.dequant_q4(words, s16, n, k, group, nibble_code=code, scale_dtype=orc.SCALE_F16)
    return DequantRef(exact, w16.astype(np.float16).astype(np.float32))


def for_plan(wf, plan: str):
    """The reference weights a launch with this plan multiplies."""
    return wf.for_plan(plan) if isinstance(wf, DequantRef) else wf
