"""Seeded input builders for the parity tests (numpy only).

Realistic per-op inputs are chained the way the reference's chain tests do (IsectTests.cpp:527-574):
projection outputs feed intersection, whose sorted output feeds the rasterizer.
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "splatx-metal_amd", "python"))
import scene  # noqa: E402


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def proj_kwargs(n=4000, C=1, seed=0, covars=False, opacities=True, aa=False, width=160, height=120, fx=150.0,
                znear=-1.0):
    r = rng(seed)
    means = np.empty((n, 3), np.float32)
    means[:, 0] = r.uniform(-2.5, 2.5, n)
    means[:, 1] = r.uniform(-2.0, 2.0, n)
    means[:, 2] = r.uniform(znear, 9.0, n)  # includes points behind / at the near plane
    q = r.standard_normal((n, 4)).astype(np.float32)  # unnormalized: the kernels normalize
    s = np.exp(r.normal(math.log(0.05), 0.8, (n, 3))).astype(np.float32)
    views = [scene.identity_view()] + [scene.jittered_view(r, 10.0, 0.5) for _ in range(C - 1)]
    kw = dict(means=means, viewmats=np.stack(views), Ks=np.stack([scene.pinhole(fx, fx * 1.1, width / 2 + 3.5,
                                                                             height / 2 - 2.25)] * C),
              width=width, height=height, calc_compensations=aa)
    if covars:
        cov = np.empty((n, 6), np.float32)
        for i in range(n):
            A = r.standard_normal((3, 3)) * 0.05
            M = A @ A.T + np.eye(3) * 1e-3
            cov[i] = [M[0, 0], M[0, 1], M[0, 2], M[1, 1], M[1, 2], M[2, 2]]
        kw["covars"] = cov
    else:
        kw["quats"], kw["scales"] = q, s
    if opacities:
        kw["opacities"] = (1.0 / (1.0 + np.exp(-r.standard_normal(n)))).astype(np.float32)
    return kw


def isect_kwargs(oracle, n=4000, seed=0, accutile=True, I=1, width=160, height=120, with_proj=False):
    """Projection outputs of `I` cameras chained into intersection inputs."""
    pk = proj_kwargs(n=n, C=I, seed=seed, width=width, height=height)
    p = oracle.projection_fused_fwd(**pk)
    kw = dict(means2d=p["means2d"], radii=p["radii"], depths=p["depths"], I=I, N=n,
              tile_width=(width + 15) // 16, tile_height=(height + 15) // 16)
    if accutile:
        kw["conics"] = p["conics"]
        kw["opacities"] = np.broadcast_to(pk["opacities"], (I, n)).copy()
    if with_proj:
        return kw, p, pk
    return kw


def raster_kwargs(oracle, n=3000, seed=0, I=1, width=150, height=100, backgrounds=False, masks=False,
                  accutile=True):
    ik, p, pk = isect_kwargs(oracle, n=n, seed=seed, accutile=accutile, I=I, width=width, height=height,
                             with_proj=True)
    it = oracle.isect_tiles(**ik)
    bits = 32 + it["tile_n_bits"] + it["image_n_bits"]
    ks, vs = oracle.sort_isect(it["isect_ids"], it["flatten_ids"], bits)
    off = oracle.isect_offset_encode(ks, I, ik["tile_width"], ik["tile_height"])
    r = rng(seed + 77)
    colors = r.uniform(0.0, 1.0, (I, n, 3)).astype(np.float32)
    opac = np.broadcast_to(pk["opacities"], (I, n)).copy()
    kw = dict(means2d=ik["means2d"], conics=p["conics"], colors=colors, opacities=opac, isect_offsets=off, flatten_ids=vs, I=I, N=n, n_isects=it["n_isects"],
              width=width, height=height, tile_width=ik["tile_width"], tile_height=ik["tile_height"])
    if backgrounds:
        kw["backgrounds"] = r.uniform(0, 1, (I, 3)).astype(np.float32)
    if masks:
        m = (r.uniform(0, 1, (I, ik["tile_height"], ik["tile_width"])) > 0.2).astype(np.uint8)
        kw["masks"] = m
    return kw


def sort_inputs(n, key_bits, seed=0, ties=True):
    r = rng(seed)
    if key_bits == 64:
        keys = r.integers(0, 2**63, n, dtype=np.uint64) * np.uint64(2) + r.integers(0, 2, n, dtype=np.uint64)
    else:
        keys = r.integers(0, 2**min(key_bits, 62), n, dtype=np.uint64)
        if key_bits > 62:
            keys |= (r.integers(0, 2, n, dtype=np.uint64) << np.uint64(key_bits - 1))
    if ties and n > 4:
        idx = r.integers(0, n, n // 3)
        keys[idx] = keys[r.integers(0, max(1, n // 50), idx.size)]
    vals = np.arange(n, dtype=np.int32)
    return keys, vals


def stable_sort_ref(keys, vals):
    order = np.argsort(keys, kind="stable")
    return keys[order], vals[order]


def make_cloud(n, cap, sh_degree, seed, logit_mu=-1.0, logit_sd=3.0, moments=True):
    """Arena arrays [cap, dim] (rows >= n zero), seeded: ~5% dead at the default logit spread."""
    r = np.random.default_rng(seed)
    dims = scene.group_dims(sh_degree)
    p = [np.zeros((cap, d), np.float32) for d in dims]
    p[0][:n] = r.normal(0, 2, (n, 3))
    p[1][:n] = r.normal(0, 1, (n, 4))
    p[2][:n] = r.normal(np.log(0.01), 0.7, (n, 3))
    p[3][:n, 0] = r.normal(logit_mu, logit_sd, n)
    p[4][:n] = r.normal(0, 0.5, (n, 3))
    if dims[5]:
        p[5][:n] = r.normal(0, 0.05, (n, dims[5]))
    m = [np.zeros((cap, d), np.float32) for d in dims]
    v = [np.zeros((cap, d), np.float32) for d in dims]
    if moments:
        for g in range(6):
            m[g][:n] = r.normal(0, 1e-3, (n, dims[g]))
            v[g][:n] = np.abs(r.normal(0, 1e-6, (n, dims[g])))
    return p, m, v
