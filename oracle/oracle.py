"""ctypes binding of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loaded only by tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline
leg, always as the checker.  ``liboracle.so`` is this build's C restatement of
the reference CPU algorithm (oracle.c); ``libfufft_ref.so`` (optional) is the
reference's own CPU sources compiled where they lie (see oracle/Makefile).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "_build" / "liboracle.so"
REF_SO = HERE / "_ref" / "libfufft_ref.so"

TW_LIBM, TW_TABLE = 0, 1
CHAIN_SINGLE, CHAIN_EVENODD, CHAIN_DIRECT = 0, 1, 2
MID = {"mul": 0, "conj": 1, "none": 2}

_i64, _i32, _vp, _d = C.c_int64, C.c_int, C.c_void_p, C.c_double


def _load_oracle() -> C.CDLL:
    L = C.CDLL(str(ORACLE_SO))
    ip = C.POINTER(C.c_int)
    L.or_factor.argtypes = [_i32, _i32, ip]
    L.or_mixedrev.argtypes = [_i32, ip, _i32]
    L.or_twiddle.argtypes = [_i32, _i32, _i32, _i32, C.POINTER(C.c_float), C.POINTER(C.c_float)]
    L.or_pass_f32.argtypes = [_vp, _i64, _i32, _i32, _i32, _i32, _i32, _i32]
    L.or_conv_f32.argtypes = [_vp, _vp, _i64, _vp, _i32, _i64, ip, ip, _i32, _i32, _i32]
    L.or_fwd_f32.argtypes = [_vp, _vp, _i32, _i64, ip, ip, _i32, _i32]
    L.or_apply_f32.argtypes = [_vp, _i64, _vp, _i64, _vp, _i32, _i64, ip, ip, _i32, _i32, _i32]
    L.or_conv_r2_f32.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp, _i32, _i64, ip, ip, _i32, _i32]
    L.or_c2c_f32.argtypes = [_vp, _vp, _i32, _i64, ip, ip, _i32, _i32, _i32]
    L.or_conv2d_f32.argtypes = [_vp, _vp, _i64, _vp, _i32, _i32, _i64, ip, ip, _i32, ip, ip,
                                _i32, _i32, _i32]
    L.or_fwd2d_f32.argtypes = [_vp, _vp, _i32, _i32, _i64, ip, ip, _i32, ip, ip, _i32, _i32]
    L.or_apply2d_f32.argtypes = [_vp, _i64, _vp, _i64, _vp, _i32, _i32, _i64, ip, ip, _i32, ip,
                                 ip, _i32, _i32, _i32]
    L.or_bfp_exponent.argtypes = [C.c_float]
    L.or_bfp_quantize.argtypes = [_vp, _i64, _i32, _vp, _vp]
    L.or_bfp_dequantize.argtypes = [_vp, _vp, _i64, _i32, _vp]
    L.or_bfp_conv.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp, _i32, _i64, _i32, ip, ip, _i32,
                              _i32, _i32]
    L.or_fft2_f64.argtypes = [_vp, _i32, _i32]
    L.or_conv_spec_f64.argtypes = [_vp, _vp, _i64, _vp, _i32, _i64, _i32]
    L.or_mixed_conv_f64.argtypes = [_vp, _vp, _vp, _i32, _i64, _i32]
    L.or_rel_l2_f32.argtypes = [_vp, _vp, _i64]
    L.or_rel_l2_f32.restype = _d
    L.or_rel_l2_f32_f64.argtypes = [_vp, _vp, _i64]
    L.or_rel_l2_f32_f64.restype = _d
    return L


lib = _load_oracle()


def load_ref() -> C.CDLL | None:
    """The reference's own CPU code, if it was built here (needs /root/reference)."""
    if not REF_SO.exists():
        return None
    R = C.CDLL(str(REF_SO))
    ip = C.POINTER(C.c_int)
    R.ref_mixed_conv_f64.argtypes = [_i32, _i32, _vp, _vp, _i64, _vp, _i64]
    R.ref_vk_chain_rev.argtypes = [_i32, ip, _i32]
    R.ref_vk_mixedrev.argtypes = [_i32, _i32, _i32]
    R.ref_vk_mixedrev16.argtypes = [_i32, _i32, _i32]
    R.ref_mixed_mixedrev.argtypes = [_i32, ip, _i32]
    R.ref_mixed_factorise.argtypes = [_i32, _i32, ip]
    for name in ("ref_vk_pipeline_v16", "ref_vk_pipeline_v16f", "ref_vk_pipeline_ip",
                 "ref_vk_pipeline_apply"):
        getattr(R, name).argtypes = [_i32, _i32, _i32, _i32, _vp, _vp, _vp, _i32]
    R.ref_vk_pipeline_fwd.argtypes = [_i32, _i32, _i32, _i32, _vp, _vp, _i32]
    R.ref_vk_c2c.argtypes = [_i32, _i32, _vp, _vp, _i32]
    R.ref_vk_conv_foursteps_cfg.argtypes = [_vp, _vp, _i32, _i32, _i32, _i32, _i32]
    R.ref_vk_conv_monolithic_cfg.argtypes = [_vp, _vp, _i32, _i32, _i32, _i32, _i32]
    R.ref_vk_conv2d.argtypes = [_i32, _i32, _vp, _vp, _vp, _i32]
    R.ref_vk_conv_r2.argtypes = [_i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _i32]
    R.ref_vk_bfp_quantize.argtypes = [_vp, _i32, _vp]
    R.ref_vk_bfp_quantize.restype = C.c_float
    R.ref_vk_v16_bfp.argtypes = [_i32, _i32, _i32, _vp, _vp, _vp, C.c_float, _vp, _vp, _i32]
    for name in ("ref_vk_main", "ref_mixed_main", "ref_inplace_main", "ref_fufft_main"):
        getattr(R, name).argtypes = []
    return R


# ---- plans ---------------------------------------------------------------------------

def _ints(xs) -> C.Array:
    return (C.c_int * max(1, len(xs)))(*xs)


class Plan:
    """Radix sequence (DIF order) and twiddle-chain mode per pass."""

    def __init__(self, radices, chains):
        self.radices = list(radices)
        self.chains = list(chains)
        self._r = _ints(self.radices)
        self._c = _ints(self.chains)

    @property
    def np(self) -> int:
        return len(self.radices)

    def __repr__(self) -> str:
        return f"Plan({self.radices}, {self.chains})"


def factor(n: int, v: int) -> list[int]:
    buf = (C.c_int * 32)()
    k = lib.or_factor(n, v, buf)
    return list(buf[:k])


def ref_plan(n: int, v: int) -> Plan:
    """The reference kernels' plan: lead radix with the single twiddle chain,
    then radix-v passes -- radix 16 with the even/odd chains (fufft.cuh:743-746),
    radix 8 with the single chain."""
    rads = factor(n, v)
    return Plan(rads, [CHAIN_EVENODD if r == 16 else CHAIN_SINGLE for r in rads])


def kernel_plan(n: int, v: int) -> Plan:
    """This build's single-launch kernel plan: the reference's chains (even/odd
    for radix 16, single otherwise); only the base twiddle source differs, and
    that is selected by the `tw` argument of the transforms."""
    return ref_plan(n, v)


def large_plan(lout: int, mid_n: int, mid_v: int = 16, ref: bool = False) -> Plan:
    """Four-step chain: lout radix-16 outer levels (single chain) + the middle."""
    m = ref_plan(mid_n, mid_v) if ref else kernel_plan(mid_n, mid_v)
    return Plan([16] * lout + m.radices, [CHAIN_SINGLE] * lout + m.chains)


def mixedrev(plan: Plan) -> np.ndarray:
    n = int(np.prod(plan.radices))
    return np.array([lib.or_mixedrev(i, plan._r, plan.np) for i in range(n)], dtype=np.int64)


# ---- transforms ------------------------------------------------------------------------

def _c64(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.complex64)


def conv(a, filt, n: int, plan: Plan, filt_stride: int = 0, mid: str = "mul",
         tw: int = TW_TABLE) -> np.ndarray:
    a = _c64(a).reshape(-1)
    f = _c64(filt).reshape(-1)
    out = np.empty_like(a)
    lib.or_conv_f32(a.ctypes.data, f.ctypes.data, filt_stride, out.ctypes.data, n, a.size // n,
                    plan._r, plan._c, plan.np, MID[mid], tw)
    return out


def fwd(a, n: int, plan: Plan, tw: int = TW_TABLE) -> np.ndarray:
    a = _c64(a).reshape(-1)
    out = np.empty_like(a)
    lib.or_fwd_f32(a.ctypes.data, out.ctypes.data, n, a.size // n, plan._r, plan._c, plan.np, tw)
    return out


def apply(spec, filt, n: int, batch: int, plan: Plan, spec_stride: int = 0,
          filt_stride: int = 0, mid: str = "mul", tw: int = TW_TABLE) -> np.ndarray:
    s = _c64(spec).reshape(-1)
    f = _c64(filt).reshape(-1)
    out = np.empty(n * batch, dtype=np.complex64)
    lib.or_apply_f32(s.ctypes.data, spec_stride, f.ctypes.data, filt_stride, out.ctypes.data, n,
                     batch, plan._r, plan._c, plan.np, MID[mid], tw)
    return out


def conv_r2(x, y, filt, n: int, plan: Plan, filt_stride: int = 0, tw: int = TW_TABLE):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    y = np.ascontiguousarray(y, dtype=np.float32).reshape(-1)
    f = _c64(filt).reshape(-1)
    u, v = np.empty_like(x), np.empty_like(y)
    lib.or_conv_r2_f32(x.ctypes.data, y.ctypes.data, f.ctypes.data, filt_stride, u.ctypes.data,
                       v.ctypes.data, n, x.size // n, plan._r, plan._c, plan.np, tw)
    return u, v


def c2c(a, n: int, plan: Plan, sign: int = -1, tw: int = TW_TABLE) -> np.ndarray:
    """Natural-order C2C: forward (sign -1) or unnormalised inverse (+1)."""
    a = _c64(a).reshape(-1)
    out = np.empty_like(a)
    lib.or_c2c_f32(a.ctypes.data, out.ctypes.data, n, a.size // n, plan._r, plan._c, plan.np,
                   sign, tw)
    return out


def conv2d(a, filt, h: int, w: int, ph: Plan, pw: Plan, filt_stride: int = 0,
           mid: str = "mul", tw: int = TW_TABLE) -> np.ndarray:
    a = _c64(a).reshape(-1)
    f = _c64(filt).reshape(-1)
    out = np.empty_like(a)
    lib.or_conv2d_f32(a.ctypes.data, f.ctypes.data, filt_stride, out.ctypes.data, h, w,
                      a.size // (h * w), ph._r, ph._c, ph.np, pw._r, pw._c, pw.np, MID[mid], tw)
    return out


def fwd2d(a, h: int, w: int, ph: Plan, pw: Plan, tw: int = TW_TABLE) -> np.ndarray:
    a = _c64(a).reshape(-1)
    out = np.empty_like(a)
    lib.or_fwd2d_f32(a.ctypes.data, out.ctypes.data, h, w, a.size // (h * w), ph._r, ph._c, ph.np,
                     pw._r, pw._c, pw.np, tw)
    return out


def apply2d(spec, filt, h: int, w: int, batch: int, ph: Plan, pw: Plan, spec_stride: int = 0,
            filt_stride: int = 0, mid: str = "mul", tw: int = TW_TABLE) -> np.ndarray:
    s = _c64(spec).reshape(-1)
    f = _c64(filt).reshape(-1)
    out = np.empty(h * w * batch, dtype=np.complex64)
    lib.or_apply2d_f32(s.ctypes.data, spec_stride, f.ctypes.data, filt_stride, out.ctypes.data, h,
                       w, batch, ph._r, ph._c, ph.np, pw._r, pw._c, pw.np, MID[mid], tw)
    return out


# ---- block floating point ------------------------------------------------------------------

def bfp_exponent(absmax: float) -> int:
    return lib.or_bfp_exponent(absmax)


def bfp_quantize(x, block: int = 64):
    x = _c64(x).reshape(-1)
    q = np.empty(2 * x.size, dtype=np.int16)
    e = np.empty(x.size // block, dtype=np.int8)
    lib.or_bfp_quantize(x.ctypes.data, x.size, block, q.ctypes.data, e.ctypes.data)
    return q, e


def bfp_dequantize(q, e, block: int = 64) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int16)
    e = np.ascontiguousarray(e, dtype=np.int8)
    x = np.empty(q.size // 2, dtype=np.complex64)
    lib.or_bfp_dequantize(q.ctypes.data, e.ctypes.data, q.size // 2, block, x.ctypes.data)
    return x


def bfp_conv(q, e, filt, n: int, plan: Plan, filt_stride: int = 0, mid: str = "mul",
             block: int = 64, tw: int = TW_TABLE):
    q = np.ascontiguousarray(q, dtype=np.int16)
    e = np.ascontiguousarray(e, dtype=np.int8)
    f = _c64(filt).reshape(-1)
    batch = q.size // (2 * n)
    qo = np.empty_like(q)
    eo = np.empty_like(e)
    lib.or_bfp_conv(q.ctypes.data, e.ctypes.data, f.ctypes.data, filt_stride, qo.ctypes.data,
                    eo.ctypes.data, n, batch, block, plan._r, plan._c, plan.np, MID[mid], tw)
    return qo, eo


# The reference's own BFP format: one fp32 scale per transform.  A restatement
# of bfp_quantize and kernel_v16_bfp (verify_kernel.cpp:1092-1135) in numpy
# float32 arithmetic (IEEE products and quotients, round to nearest even):
#   mx = max(abs-max of re and im, 1e-30); inv = 32767 / mx;
#   q = rint(clamp(x * inv, -32767, 32767)); scale = mx / 32767; x = q * scale.
# The conv dequantises signal and filter, runs the fp32 pipeline (conv above,
# whose multiply takes the dequantised filter value) and quantises the result
# per transform.  Pinned bit for bit to the compiled reference in
# tests/test_oracle_pins.py and by tests/golden/bfp_scaled_*.npz.

def bfp_scaled_quantize(x, n: int):
    x = _c64(x).reshape(-1, n)
    parts = x.view(np.float32).reshape(x.shape[0], 2 * n)
    mx = np.maximum(np.abs(parts).max(axis=1), np.float32(1e-30)).astype(np.float32)
    inv = (np.float32(32767.0) / mx).astype(np.float32)
    y = np.clip(parts * inv[:, None], np.float32(-32767.0), np.float32(32767.0))
    return np.rint(y).astype(np.int16).reshape(-1), (mx / np.float32(32767.0)).astype(np.float32)


def bfp_scaled_dequantize(q, scale, n: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int16).reshape(-1, 2 * n).astype(np.float32)
    s = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1, 1)
    return np.ascontiguousarray((q * s).astype(np.float32)).view(np.complex64).reshape(-1)


def bfp_scaled_conv(q, scale, fq, fscale, n: int, plan: Plan, filt_stride: int = 0, mid: str = "mul",
                    tw: int = TW_TABLE):
    a = bfp_scaled_dequantize(q, scale, n)
    f = bfp_scaled_dequantize(fq, fscale, n) if fq is not None else np.zeros(n, np.complex64)
    return bfp_scaled_quantize(conv(a, f, n, plan, filt_stride=filt_stride, mid=mid, tw=tw), n)


# ---- fp64 ------------------------------------------------------------------------------------

def conv_spec_f64(a, spec_nat, n: int, spec_stride: int = 0, mid: str = "mul") -> np.ndarray:
    """fp64 truth: IDFT(DFT(a) mid spec) with the natural-order spectrum spec."""
    a = _c64(a).reshape(-1)
    s = _c64(spec_nat).reshape(-1)
    out = np.empty(a.size, dtype=np.complex128)
    lib.or_conv_spec_f64(a.ctypes.data, s.ctypes.data, spec_stride, out.ctypes.data, n,
                         a.size // n, MID[mid])
    return out


def fft2_f64(x, sign: int) -> np.ndarray:
    y = np.ascontiguousarray(x, dtype=np.complex128).copy()
    lib.or_fft2_f64(y.ctypes.data, y.size, sign)
    return y


def mixed_conv_f64(a, spec_dr, n: int, v: int = 16) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.complex128).reshape(-1)
    s = np.ascontiguousarray(spec_dr, dtype=np.complex128).reshape(-1)
    out = np.empty_like(a)
    lib.or_mixed_conv_f64(a.ctypes.data, s.ctypes.data, out.ctypes.data, n, a.size // n, v)
    return out


def rel_l2(x, y) -> float:
    x = np.asarray(x, dtype=np.complex128).reshape(-1)
    y = np.asarray(y, dtype=np.complex128).reshape(-1)
    den = np.sum(np.abs(y) ** 2)
    num = np.sum(np.abs(x - y) ** 2)
    return float(np.sqrt(num / den)) if den > 0 else float(np.sqrt(num))
