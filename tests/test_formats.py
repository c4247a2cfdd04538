"""Formats either side of the step, host side (no GPU): the PLY reader and the SXCK header /
fingerprint checks of libsplatx_hip.so against the reference's own PlyIO.cpp and Checkpoint.cpp
(built in place under oracle/_ref; skipped where the reference tree is absent).

- read_inria_ply: files written by the reference's write_inria_ply (degrees 0-3, padded and not)
  read back identically (arrays bit for bit, count, inferred degree); malformed files fail as the
  reference's reader does.
- load_checkpoint_header / verify_checkpoint_config: same header fields and same error messages for
  every corruption and every fingerprint mismatch.
"""
import struct

import numpy as np
import pytest

import splatx_hip as sh
from inputs import make_cloud


def same(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.mark.parametrize("deg,pad", [(0, True), (1, True), (1, False), (2, True), (3, True)])
def test_ply_read_matches_reference(reference, tmp_path, deg, pad):
    n = 700
    p, _, _ = make_cloud(n, n, deg, 30 + deg)
    p[0][5, 1] = np.nan  # a non-finite row the filter drops
    path = str(tmp_path / "c.ply")
    st = reference.export_ply(p, n, deg, path, pad_sh_full=pad)
    assert st["removed_nonfinite"] == 1 and st["kept"] > 0
    mine = sh.ply_read(path)
    ref = reference.read_ply(path, n)
    assert mine["count"] == ref["count"] == st["kept"]
    assert mine["sh_degree"] == ref["sh_degree"] == (3 if pad and deg > 0 else deg)
    for g in range(6):
        assert same(mine["params"][g], ref["params"][g]), g


def _write_ply(path, header_lines, body=b""):
    with open(path, "wb") as f:
        f.write(("\n".join(header_lines) + "\n").encode())
        f.write(body)


def test_ply_read_errors(reference, tmp_path):
    props = ["property float " + n for n in ("x", "y", "z", "f_dc_0", "f_dc_1", "f_dc_2", "opacity", "scale_0",
                                             "scale_1", "scale_2", "rot_0", "rot_1", "rot_2", "rot_3")]
    cases = {
        "ascii": ["ply", "format ascii 1.0", "element vertex 1"] + props + ["end_header"],
        "uchar": ["ply", "format binary_little_endian 1.0", "element vertex 1"] + props + ["property uchar red",
                                                                                          "end_header"],
        "missing": ["ply", "format binary_little_endian 1.0", "element vertex 1"] + props[1:] + ["end_header"],
        "rest4": ["ply", "format binary_little_endian 1.0", "element vertex 1"] + props +
                 [f"property float f_rest_{i}" for i in range(4)] + ["end_header"],
        "truncated": ["ply", "format binary_little_endian 1.0", "element vertex 3"] + props + ["end_header"],
        "noheader": ["ply", "format binary_little_endian 1.0"],
    }
    for name, lines in cases.items():
        path = str(tmp_path / f"{name}.ply")
        body = struct.pack("<14f", *range(14)) if name in ("truncated", "missing") else b""
        _write_ply(path, lines, body)
        with pytest.raises(sh.SxRuntimeError) as mine:
            sh.ply_read(path)
        with pytest.raises(sh.SxRuntimeError) as ref:
            reference.read_ply(path, 8)
        assert str(mine.value) == str(ref.value), name
    with pytest.raises(sh.SxRuntimeError):
        sh.ply_read(str(tmp_path / "absent.ply"))


def _ckpt(reference, tmp_path, fp16=False, n=300, deg=2, **cfg_kw):
    p, m, v = make_cloud(n, n, deg, 40)
    cfg = sh.CkptConfig.make(sh_degree=deg, total_iters=3000, **cfg_kw)
    path = str(tmp_path / ("c16.sxck" if fp16 else "c32.sxck"))
    reference.save_checkpoint(cfg, 123, p, m, v, n, deg, path, rng_state="1 2 3" if cfg.mcmc_enabled else None,
                              fp16=fp16)
    return path, cfg


@pytest.mark.parametrize("fp16", [False, True])
def test_checkpoint_header_matches_reference(reference, tmp_path, fp16):
    path, cfg = _ckpt(reference, tmp_path, fp16, mcmc_enabled=1, cap_max=500, mcmc_seed=42, factor=2, test_split=8,
                      antialiased=1, scene_scale=1.5, ssim_weight=0.2)
    mine = sh.checkpoint_read_header(path)
    ref = reference.load_checkpoint(path, 300)["header"]
    assert mine == ref
    assert mine["iter"] == 123 and mine["alive_count"] == 300 and mine["fp16"] == int(fp16)


def test_checkpoint_header_corruptions(reference, tmp_path):
    path, _ = _ckpt(reference, tmp_path)
    good = open(path, "rb").read()
    edits = {
        "magic": lambda b: b"XXCK" + b[4:],
        "version": lambda b: b[:4] + struct.pack("<I", 2) + b[8:],
        "flags": lambda b: b[:8] + struct.pack("<I", 6) + b[12:],
        "reserved": lambda b: b[:30] + b"\x01" + b[31:],
        "degree": lambda b: b[:12] + struct.pack("<i", 5) + b[16:],
        "iter": lambda b: b[:56] + struct.pack("<i", -1) + b[60:],
        "count": lambda b: b[:60] + struct.pack("<q", 0) + b[68:],
        "short": lambda b: b[:20],
    }
    # field offsets: magic 0, version 4, flags 8, sh_degree 12, factor 16, test_split 20, total_iters
    # 24, mcmc 28, antialiased 29, reserved 30, pad 31, cap_max 32, seed 40, scene_scale 48,
    # ssim_weight 52, iter 56, alive_count 60, rng length 68
    for name, f in edits.items():
        bad = str(tmp_path / f"{name}.sxck")
        open(bad, "wb").write(f(good))
        with pytest.raises(sh.SxRuntimeError) as mine:
            sh.checkpoint_read_header(bad)
        with pytest.raises(sh.SxRuntimeError) as ref:
            reference.load_checkpoint(bad, 300)
        assert str(mine.value) == str(ref.value), (name, mine.value, ref.value)


def test_verify_config_matches_reference(reference):
    base = dict(sh_degree=3, factor=2, test_split=8, total_iters=30000, mcmc_enabled=1, antialiased=0, cap_max=1000,
                mcmc_seed=42, scene_scale=1.25, ssim_weight=0.2)
    saved = sh.CkptConfig.make(**base)
    sh.checkpoint_verify_config(saved, sh.CkptConfig.make(**base))
    changes = dict(sh_degree=2, factor=4, test_split=0, total_iters=100, mcmc_enabled=0, antialiased=1, cap_max=5,
                   mcmc_seed=7, scene_scale=1.5, ssim_weight=0.0)
    for k, val in changes.items():
        cur = sh.CkptConfig.make(**dict(base, **{k: val}))
        with pytest.raises(sh.SxRuntimeError) as mine:
            sh.checkpoint_verify_config(saved, cur)
        with pytest.raises(sh.SxRuntimeError) as ref:
            reference.checkpoint_verify_config(saved, cur)
        assert str(mine.value) == str(ref.value), k
