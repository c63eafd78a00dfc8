"""Cost-model calibration on the MI355X (solutions/calibrate.py semantics): the kernel counter sees the
native launches, and a small-grid calibration of a small model produces a usable record whose models
predict the measured packed steps."""

from __future__ import annotations

import pytest
import torch

from conftest import small_cfg, to_model_config

pytestmark = pytest.mark.gpu


def test_count_kernels_sees_native_launches(cuda):
    from thesis_amd import _lsk
    from thesis_amd.solutions.calibrate import count_kernels

    src = torch.zeros(4, 16, dtype=torch.uint8, device=cuda)
    dst = torch.empty_like(src)
    assert count_kernels(lambda: _lsk.copy_rows(dst, None, src, None, 4)) == 1
    assert count_kernels(lambda: [_lsk.copy_rows(dst, None, src, None, 4) for _ in range(3)]) == 3


def test_small_calibration_record(cuda, tmp_path):
    from thesis_amd.common.model import LayerSkipLlama
    from thesis_amd.solutions.calibrate import calibrate
    from thesis_amd.solutions.cost_model import RooflineCostModel, load_cost_model, save_json

    mcfg = to_model_config(small_cfg())
    model = LayerSkipLlama.random(mcfg, seed=0, dtype=torch.bfloat16, max_seq=1024)
    res = calibrate(model, "small", do_validate=True, k=2, ns=(1, 4, 16, 64, 128),
                    grid=dict(Bs=(1, 4), Ts=(1, 4), ctxs=(128, 256)),
                    val=dict(ctxs=(128,), Bs=(1, 4), Ts=(2, 4), prefill=(64,)),
                    bw_shape=(4096, 1024), mm=1024, log=lambda s: None)
    g = res["gpu"]
    print(f"bw {g.bw:.3g} B/ms flops {g.flops:.3g} flops_eff {g.flops_eff:.3g} t_op {g.t_op * 1e3:.2f} us "
          f"knee {g.knee_measured} n_op {g.n_op_layer}/{g.n_op_bucket}/{g.n_op_head}/{g.n_op_segment}")
    assert g.bw > 0 and g.flops > 0 and g.flops_eff > 0 and 0 < g.t_op < 0.1
    # one packed layer launches at least norm, qkv, rope+append, attention, o, norm, w13, w2
    assert g.n_op_layer >= 8 and g.n_op_head >= 2
    assert 4 <= g.knee_measured < 128
    assert len(res["linear_grid"]) == 8 and res["linear"]["a"] > 0
    v = res["validation"]
    assert v["roofline_all"]["n"] == 7 and v["linear_all"]["n"] == 7 and v["roofline_prefill"]["n"] == 1
    p = tmp_path / "small.json"
    save_json(p, res)
    cm = load_cost_model(p, mcfg)
    assert isinstance(cm, RooflineCostModel) and cm.F == g.flops_eff
    assert float(cm.t_sh(4, 2, 512)) > 0
