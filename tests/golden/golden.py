"""Golden fixtures: inputs and outputs of the reference's own CPU transcription
of its kernels (verify_kernel.cpp, compiled where it lies into oracle/_ref by
oracle/Makefile), written by make_golden.py.  The reference stores no vectors
of its own; these pin the oracle where /root/reference is absent.

Each fixture is an .npz holding the case parameters, the inputs, and the
reference outputs; replay() recomputes the outputs with the oracle in
libm-twiddle mode (the reference's twiddle source), which must agree bit for
bit.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

from oracle import oracle as O

HERE = Path(__file__).resolve().parent


def load_all() -> dict:
    return {p.stem: dict(np.load(p, allow_pickle=False)) for p in sorted(HERE.glob("*.npz"))}


def replay(case: dict) -> dict:
    kind = str(case["kind"])
    if kind == "v16":
        n = int(case["n"])
        return {"out": O.conv(case["a"], case["bdr"], n, O.ref_plan(n, 16), filt_stride=n, tw=O.TW_LIBM)}
    if kind == "r8":
        n = int(case["n"])
        return {"out": O.conv(case["a"], case["bdr"], n, O.ref_plan(n, 8), filt_stride=n, tw=O.TW_LIBM)}
    if kind == "split":
        n = int(case["n"])
        plan = O.ref_plan(n, 8)
        spec = O.fwd(case["a"], n, plan, tw=O.TW_LIBM)
        out = O.apply(spec, case["bdr"], n, spec.size // n, plan, spec_stride=n, filt_stride=n, tw=O.TW_LIBM)
        return {"spec": spec, "out": out}
    if kind == "conv2d":
        h, w = int(case["h"]), int(case["w"])
        return {"out": O.conv2d(case["a"], case["bdr"], h, w, O.ref_plan(h, 8), O.ref_plan(w, 8),
                                filt_stride=h * w, tw=O.TW_LIBM)}
    if kind == "r2":
        n = int(case["n"])
        u, v = O.conv_r2(case["x"], case["y"], case["bdr"], n, O.ref_plan(n, 8), filt_stride=n, tw=O.TW_LIBM)
        return {"u": u, "v": v}
    if kind == "fourstep":
        n, lout, mid = int(case["n"]), int(case["lout"]), int(case["mid"])
        mid_v = int(case["mid_v"]) if "mid_v" in case else 16
        plan = O.large_plan(lout, mid, mid_v, ref=True)
        return {"out": O.conv(case["a"], case["bdr"], n, plan, filt_stride=n, tw=O.TW_LIBM)}
    if kind == "bfp_scaled":
        n = int(case["n"])
        oq, osc = O.bfp_scaled_conv(case["aq"], case["asc"], case["bq"], case["bsc"], n, O.ref_plan(n, 16),
                                    tw=O.TW_LIBM)
        return {"oq": oq, "osc": osc}
    if kind == "c2c_stockham":
        # the reference's Stockham C2C rounds in a different order from this
        # build's DIF + permutation: no bit-exact outputs; test_oracle_c2c
        # checks it to fp32 rounding
        return {}
    raise ValueError(kind)
