"""SXT1 fixture reader and the reference's comparison helpers.

Format (Sources/SplatXCore/include/splatx/SXTensor.h:8-26): "SXT1" | u32 dtype | u32 ndim |
u64 shape[ndim] | little-endian payload; dtype 0=float32, 1=int32, 3=uint8.
`assert_all_close` follows TestHarness.h:90-149: tolerances come only from meta.json, NaN always
fails, zero compared elements fails, optional rel_l2 is checked too.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np

FIXTURES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures")
_DT = {0: np.float32, 1: np.int32, 3: np.uint8}


def load(path: str) -> np.ndarray:
    with open(path, "rb") as f:
        raw = f.read()
    if raw[:4] != b"SXT1":
        raise ValueError(f"bad magic in {path}")
    dtype, ndim = struct.unpack_from("<II", raw, 4)
    shape = struct.unpack_from("<" + "Q" * ndim, raw, 12)
    off = 12 + 8 * ndim
    return np.frombuffer(raw, dtype=_DT[dtype], offset=off, count=int(np.prod(shape, dtype=np.int64))).reshape(shape).copy()


def fx(d: str, name: str) -> np.ndarray:
    return load(os.path.join(FIXTURES, d, name if name.endswith(".sxt") else name + ".sxt"))


def meta(d: str) -> dict:
    with open(os.path.join(FIXTURES, d, "meta.json")) as f:
        return json.load(f)


def has(d: str, name: str) -> bool:
    return os.path.exists(os.path.join(FIXTURES, d, name + ".sxt"))


def u64_from_lohi(lo: np.ndarray, hi: np.ndarray) -> np.ndarray:
    return (hi.astype(np.uint32).astype(np.uint64) << np.uint64(32)) | lo.astype(np.uint32).astype(np.uint64)


def assert_all_close(actual, expected, m: dict, tensor: str, mask=None):
    tol = m["tolerances"][tensor]
    rtol, atol = tol["rtol"], tol["atol"]
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    assert a.size == e.size, f"{tensor}: size {a.size} != {e.size}"
    if mask is not None:
        mk = np.asarray(mask).ravel().astype(bool)
        period = a.size // mk.size
        sel = np.repeat(mk, period)
        a, e = a[sel], e[sel]
    assert a.size > 0, f"{tensor}: compared 0 elements"
    d = np.abs(a - e)
    bad = ~(d <= atol + rtol * np.abs(e))
    assert not bad.any(), (f"{tensor}: allclose violated {int(bad.sum())}/{a.size} (rtol={rtol} atol={atol}); "
                           f"worst idx {int(np.argmax(np.where(bad, d, -1)))}")
    if "rel_l2" in tol:
        ref2 = float((e * e).sum())
        rel = np.sqrt(float((d * d).sum()) / ref2) if ref2 > 0 else np.sqrt(float((d * d).sum()))
        assert rel <= tol["rel_l2"], f"{tensor}: rel_l2 {rel} > {tol['rel_l2']}"


def rel_l2(a, e) -> float:
    a = np.asarray(a, np.float64).ravel()
    e = np.asarray(e, np.float64).ravel()
    den = float((e * e).sum())
    num = float(((a - e) ** 2).sum())
    return float(np.sqrt(num / den)) if den > 0 else float(np.sqrt(num))
