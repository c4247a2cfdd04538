"""The caller loop's host side (no GPU): the C and ctypes layouts of its structs agree, its schedule
defaults are the reference's TrainConfig / McmcOptions defaults, and sxh_train_plan_at — the
per-iteration step arguments the loop forms — equals the reference's own means_lr_at, sh_degree_at
and Trainer::mcmc_refine_due bit for bit (oracle/_ref, built from the reference tree; skipped where
it is absent), over whole schedules at several lengths and ratios."""
import ctypes as C
import math
import os
import subprocess

import numpy as np
import pytest

import splatx_hip as sh

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

STRUCTS = {
    "sxh_train_camera": sh.TrainCamera,
    "sxh_train_schedule": sh.TrainSchedule,
    "sxh_train_plan": sh.TrainPlan,
    "sxh_train_progress": sh.TrainProgress,
    "sxh_splat_snapshot": sh.SplatSnapshot,
    "sxh_train_loop_args": sh.TrainLoopArgs,
    "sxh_train_loop_result": sh.TrainLoopResult,
}


def test_struct_layouts_match_the_header(tmp_path):
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "splatx_hip.h"', "int main(void) {"]
    for cname, py in STRUCTS.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'printf("{cname}.{f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], check=True, capture_output=True,
                                                         text=True).stdout.splitlines())
    for cname, py in STRUCTS.items():
        assert int(got[cname]) == C.sizeof(py), cname
        for f, _ in py._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(py, f).offset, (cname, f)


def test_schedule_defaults_are_the_references(reference):
    ours = sh.train_schedule_defaults()
    ref = reference.train_defaults()
    for k, v in ref.items():
        mine = getattr(ours, k)
        assert float(mine) == (v if k in ("total_iters", "cap_max", "mcmc_seed") else float(np.float32(v))), k
    assert ours.mcmc_enabled == 0


SCHEDULES = [
    dict(total_iters=300, scene_scale=1.0, lr_means=1.6e-4, sh_degree_interval_ratio=1 / 30, mcmc_enabled=1,
         refine_start_ratio=500 / 30000, refine_stop_ratio=25000 / 30000, refine_every_ratio=100 / 30000),
    dict(total_iters=30000, scene_scale=2.37, lr_means=1.6e-4, sh_degree_interval_ratio=1 / 30, mcmc_enabled=1,
         refine_start_ratio=500 / 30000, refine_stop_ratio=25000 / 30000, refine_every_ratio=100 / 30000),
    dict(total_iters=7, scene_scale=0.5, lr_means=3e-3, sh_degree_interval_ratio=0.3, mcmc_enabled=1,
         refine_start_ratio=0.1, refine_stop_ratio=0.95, refine_every_ratio=0.2),
    dict(total_iters=1234, scene_scale=1.0, lr_means=1.6e-4, sh_degree_interval_ratio=0.0001, mcmc_enabled=0,
         refine_start_ratio=0.0, refine_stop_ratio=1.0, refine_every_ratio=0.01),
]


@pytest.mark.parametrize("k", range(len(SCHEDULES)))
@pytest.mark.parametrize("sh_degree", [0, 3])
def test_train_plan_matches_reference_schedule(reference, k, sh_degree):
    cfg = SCHEDULES[k]
    s = sh.train_schedule_defaults()
    for f, v in cfg.items():
        setattr(s, f, v)
    T = cfg["total_iters"]
    iters = np.unique(np.concatenate([np.arange(0, min(T + 5, 3000)), np.linspace(0, T + 10, 997).astype(int),
                                      np.array([T - 1, T, T + 1])]))
    lr0, deg, due = reference.train_plans(T, cfg["scene_scale"], cfg["lr_means"], cfg["sh_degree_interval_ratio"],
                                          cfg["mcmc_enabled"], cfg["refine_start_ratio"], cfg["refine_stop_ratio"],
                                          cfg["refine_every_ratio"], sh_degree, iters)
    count = 12345
    for j, it in enumerate(iters):
        p = sh.train_plan_at(s, int(it), sh_degree, count)
        assert np.float32(p.lr[0]).view(np.uint32) == lr0[j].view(np.uint32), (it, p.lr[0], lr0[j])
        assert p.degrees_to_use == deg[j], it
        assert p.refine_due == due[j], it
        assert p.inject_noise == (1 if cfg["mcmc_enabled"] and not due[j] else 0)
        assert list(p.lr)[1:] == [s.lr_quats, s.lr_scales, s.lr_opacities, s.lr_sh0, s.lr_shN]
    assert due.any() == bool(cfg["mcmc_enabled"])  # every schedule here has refine iterations when MCMC is on


def test_train_plan_regularization_weights_and_noise():
    s = sh.train_schedule_defaults()
    s.opacity_reg, s.scale_reg, s.mcmc_enabled = 0.01, 0.02, 1
    for count in (1, 7, 1_000_000, 3_999_999):
        p = sh.train_plan_at(s, 42, 3, count)
        # Trainer.cpp:933-940: reg / float(N) and reg / float(N * 3), in float
        assert p.opacity_reg_w == np.float32(np.float32(0.01) / np.float32(count))
        assert p.scale_reg_w == np.float32(np.float32(0.02) / np.float32(count * 3))
        # noise_scale = means_lr_at(iter) * noise_lr in float (mcmc.py:190)
        assert p.noise_scale == np.float32(np.float32(p.lr[0]) * np.float32(5e5))
    s.opacity_reg = s.scale_reg = 0.0
    p = sh.train_plan_at(s, 42, 3, 10)
    assert p.opacity_reg_w == 0.0 and p.scale_reg_w == 0.0
    with pytest.raises(sh.SxInvalidArgument):
        sh.train_plan_at(s, 1, 3, 0)
    assert math.isfinite(p.noise_scale)
