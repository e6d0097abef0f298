"""Drift of a 32-layer stack through the fused op (bf16 on the GPU) against
the same stack in fp32 on the CPU oracle; window layers everywhere except
full attention at layers 7/15/23/31, residual add between layers.

The bar: at every layer the GPU stack's relative drift stays within 1.5x
(+2e-3) of the drift of the oracle's bf16 rounding model (the same rounding
points evaluated exactly on the CPU), i.e. the fused kernel adds no error
beyond what bf16 storage of Q_rot, K_rot, P and the activations implies.
The full-size cfg2 stack is reported by ``bench.py --drift``.
"""
import math

import pytest

pytestmark = pytest.mark.gpu


def test_drift_stack_cfg0(device):
    import bench
    rep = bench.drift_stack("cfg0", device, layers=32)
    assert len(rep["per_layer"]) == 32
    for r in rep["per_layer"]:
        assert math.isfinite(r["gpu_rel"]), r
        assert r["gpu_rel"] <= 1.5 * r["bf16_model_rel"] + 2e-3, r
    print(f"final relative drift: gpu {rep['final_gpu_rel']:.3e}, bf16 model {rep['final_bf16_model_rel']:.3e}")
