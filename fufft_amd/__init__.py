"""fuFFT for MI355X: Python binding of the C ABI in include/fufft/fufft.h.

The compute path is the in-tree HIP library ``libfufft_amd.so`` (built by
``fufft_amd.build``).  There is no fallback: if the library is missing, import
fails loudly.  Device buffers are torch tensors on ``cuda`` (ROCm); every
launch wrapper checks their dtype, contiguity, size and device before the
call (``_dev``), and launches on torch's current stream unless given one.

torch is imported before the library is loaded so that both share torch's HIP
runtime (torch bundles its own ``libamdhip64.so.7``; the loader then resolves
the library's dependency to that same copy).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

try:  # must precede loading the HIP library, see module docstring
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - torch is part of the image
    torch = None

_LIB_PATH = Path(__file__).resolve().parent / "libfufft_amd.so"

ABI_VERSION = 4                   # FUFFT_ABI_VERSION of the header this binding follows
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP, ERR_ALIGN, ERR_SCRATCH = 0, -1, -2, -3, -4, -5
SCRATCH_BYTES = 64 << 20          # FUFFT_SCRATCH_BYTES
MID = {"mul": 0, "conj": 1, "none": 2}
VARIANT = {"v16": 0, "r8": 1, "auto": 2}
LAYOUT = {"dr": 0, "lane": 1, "bperm": 2}
FILTER_SPECTRUM, FILTER_TAPS = 0, 1
FORWARD, INVERSE = -1, 1
BFP_BLOCK = 64
VALUES_PER_LANE = {"v16": 16, "r8": 8}


def resolve_variant(n: int, variant: str) -> str:
    """The lane layout FUFFT_AUTO picks for n (mirrors the library's rule: the
    faster one with a digit-order filter, fastest_variant(n, "dr"))."""
    if variant != "auto":
        return variant
    return "r8" if n in (512, 4096, 8192) else "v16"


def fastest_variant(n: int, layout: str = "lane") -> str:
    """The faster variant for an n-point conv whose filter is in `layout`
    (fufft_fastest_variant): with "lane", "r8" at n = 512 and "v16" from
    n = 1024 on.  Plan the filter and launch with it."""
    v = lib.fufft_fastest_variant(n, LAYOUT[layout])
    if v < 0:
        raise FufftError(v, "fufft_fastest_variant")
    return "r8" if v == VARIANT["r8"] else "v16"


class FufftError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: {lib.fufft_status_string(status).decode()} ({status})")


def _load() -> C.CDLL:
    if not _LIB_PATH.exists():
        raise FileNotFoundError(
            f"{_LIB_PATH} is missing: build it with `python fufft_amd/build.py` "
            "(there is no CPU fallback)")
    L = C.CDLL(str(_LIB_PATH))
    i64, i32, vp, fp = C.c_int64, C.c_int, C.c_void_p, C.POINTER(C.c_float)
    sig = {
        "fufft_abi_version": ([], i32),
        "fufft_init": ([i32], i32),
        "fufft_status_string": ([i32], C.c_char_p),
        "fufft_supported": ([i64, i32], i32),
        "fufft_fastest_variant": ([i64, i32], i32),
        "fufft_mid_reads_filter": ([i32], i32),
        "fufft_plan_radices": ([i64, i32, C.POINTER(C.c_int)], i32),
        "fufft_digit_order": ([i64, i32, C.POINTER(C.c_int32)], i32),
        "fufft_plan_chains": ([i64, i32, C.POINTER(C.c_int)], i32),
        "fufft_plan_filter_f32": ([i64, i32, i32, i32, i32, vp, vp], i32),
        "fufft_twiddle_table_host": ([i32, vp], i32),
        "fufft_twiddle_table_host_source": ([i32, i32, vp], i32),
        "fufft_set_twiddles": ([i32, i32], i32),
        "fufft_get_twiddles": ([i32, C.POINTER(C.c_int)], i32),
        "fufft_conv_f32": ([vp, vp, i64, vp, i64, i64, i32, i32, i32, vp], i32),
        "fufft_fwd_f32": ([vp, vp, i64, i64, i32, vp], i32),
        "fufft_apply_f32": ([vp, i64, vp, i64, vp, i64, i64, i32, i32, i32, vp], i32),
        "fufft_conv_r2_f32": ([vp, vp, vp, i64, vp, vp, i64, i64, i32, i32, vp], i32),
        "fufft_bfp_exponent": ([C.c_float], i32),
        "fufft_bfp_quantize": ([vp, i64, i64, vp, vp], i32),
        "fufft_bfp_dequantize": ([vp, vp, i64, i64, vp], i32),
        "fufft_conv_bfp16": ([vp, vp, vp, i64, vp, vp, i64, i64, i64, i32, i32, i32, vp], i32),
        "fufft_conv_bfp16_scaled": ([vp, vp, vp, vp, i64, vp, vp, i64, i64, i32, i32, i32, vp], i32),
        "fufft_bfp_scaled_quantize": ([vp, i64, i64, vp, vp], i32),
        "fufft_bfp_scaled_dequantize": ([vp, vp, i64, i64, vp], i32),
        "fufft_large_plan": ([i64, C.POINTER(C.c_int), C.POINTER(C.c_int)], i32),
        "fufft_large_digit_order": ([i64, i32, C.POINTER(C.c_int32)], i32),
        "fufft_plan_filter_large_f32": ([i64, i32, i32, i32, vp, vp], i32),
        "fufft_conv_large_f32": ([vp, vp, i64, i64, i64, i32, i32, vp], i32),
        "fufft_plan2d": ([i64, i64, C.POINTER(C.c_int), C.POINTER(C.c_int)], i32),
        "fufft_plan2d_column_order": ([i64, i64, C.POINTER(C.c_int32)], i32),
        "fufft_plan_filter2d_f32": ([i64, i64, i32, i32, i32, vp, vp], i32),
        "fufft_conv2d_f32": ([vp, vp, i64, vp, i64, i64, i64, i32, i32, vp], i32),
        "fufft_conv2d_r2_f32": ([vp, vp, vp, i64, vp, vp, vp, i64, i64, i64, i32, vp], i32),
        "fufft_conv2d_r2_noalloc_f32": ([vp, vp, vp, i64, vp, vp, i64, i64, i64, i32, vp], i32),
        "fufft_fwd2d_f32": ([vp, vp, i64, i64, i64, vp], i32),
        "fufft_apply2d_f32": ([vp, i64, vp, i64, vp, i64, i64, i64, i32, i32, vp], i32),
        "fufft_c2c_f32": ([vp, vp, i64, i64, i32, i32, vp], i32),
        "fufft_stream_f32": ([vp, vp, i64, i32, vp], i32),
        "fufft_stream_shape_f32": ([vp, vp, i64, i32, i32, i32, i32, i32, i32, i32, vp], i32),
        "fufft_transforms_per_workgroup": ([i64, i32], i32),
        "fufft_conv_timed_f32": ([vp, vp, i64, vp, i64, i64, i32, i32, i32, vp, i64, vp], i32),
        "fufft_plan_filter_device_f32": ([vp, vp, i64, i64, i32, i32, i32, i32, vp], i32),
        "fufft_plan_filter_large_device_f32": ([vp, vp, i64, i64, i32, i32, i32, vp], i32),
        "fufft_plan_filter2d_device_f32": ([vp, vp, i64, i64, i64, i32, i32, i32, vp], i32),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name, None)
        if f is None:
            continue
        f.argtypes, f.restype = args, res
    # a library built from another header would take these arguments wrongly
    abi = L.fufft_abi_version() if hasattr(L, "fufft_abi_version") else None
    if abi != ABI_VERSION:
        raise ImportError(f"{_LIB_PATH} has ABI version {abi}, this binding expects {ABI_VERSION}: "
                          "rebuild it with `python fufft_amd/build.py`")
    return L


lib = _load()


def check(status: int, where: str) -> None:
    if status != OK:
        raise FufftError(status, where)


# Element types accepted for each kind of buffer (checked before any launch).
_DT = {}
if torch is not None:
    _DT = {
        "complex": (torch.complex64, torch.float32),          # interleaved (re, im) fp32
        "real": (torch.float32,),
        "bfp": (torch.int16, torch.int32),                    # int16 pairs, 4 bytes per point
        "exp": (torch.int8, torch.uint8),
        "scale": (torch.float32,),
        "words": (torch.int32,),
    }


def _check_shape(x, name: str, nbytes: int, kind: str) -> None:
    if torch is None or not isinstance(x, torch.Tensor):
        raise TypeError(f"{name}: expected a torch tensor in GPU memory, got {type(x).__name__}")
    if x.dtype not in _DT[kind]:
        allowed = ", ".join(str(d) for d in _DT[kind])
        raise ValueError(f"{name}: dtype {x.dtype} is not one of {allowed}")
    if not x.is_contiguous():
        raise ValueError(f"{name}: tensor is not contiguous")
    have = x.numel() * x.element_size()
    if have < nbytes:
        raise ValueError(f"{name}: holds {have} bytes, the call reads or writes {nbytes}")


def _check_device(x, name: str) -> None:
    if not x.is_cuda:
        raise ValueError(f"{name}: tensor is on {x.device}, not in GPU memory")
    if x.device.index != torch.cuda.current_device():
        raise ValueError(f"{name}: tensor is on {x.device}, the current device is "
                         f"cuda:{torch.cuda.current_device()}")


def _ptrs(*specs) -> list:
    """Device addresses for a launch.  Each spec is (tensor, name, nbytes,
    kind), or None for an argument the call does not read.  Every tensor is
    checked first for type, dtype (kind), contiguity and size (at least
    nbytes), then every tensor for its device (the current GPU), so a host
    array, a wrong dtype or a short buffer raises TypeError / ValueError here
    and never becomes an out-of-bounds device access."""
    for sp in specs:
        if sp is not None:
            _check_shape(*sp)
    for sp in specs:
        if sp is not None:
            _check_device(sp[0], sp[1])
    return [None if sp is None else sp[0].data_ptr() for sp in specs]


def _count(stride: int, n: int, batch: int, name: str) -> int:
    """Items an array of per-transform stride `stride` must hold (0 = one shared)."""
    if stride == 0:
        return 1
    if stride == n:
        return max(batch, 1)
    raise ValueError(f"{name}: stride {stride} is neither 0 (shared) nor {n} (one per transform)")


def _stream(stream) -> int:
    """hipStream_t for a launch: an explicit torch stream or raw handle, else
    torch's current stream (so launches order with the caller's torch work)."""
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


# ---- host planning ---------------------------------------------------------------
# Every variant argument defaults to "auto" (FUFFT_AUTO), in the planners and
# the launches alike, so a filter planned with the defaults always matches a
# launch made with the defaults.

def init(device: int = 0) -> None:
    check(lib.fufft_init(device), "fufft_init")


def supported(n: int, variant: str = "auto") -> bool:
    return bool(lib.fufft_supported(n, VARIANT[variant]))


def plan_radices(n: int, variant: str = "auto") -> list[int]:
    buf = (C.c_int * 64)()
    np_ = lib.fufft_plan_radices(n, VARIANT[variant], buf)
    if np_ < 0:
        raise FufftError(np_, "fufft_plan_radices")
    return list(buf[:np_])


def plan_chains(n: int, variant: str = "auto") -> list[int]:
    """Per pass: 0 single twiddle chain, 1 radix-16 even/odd chains."""
    buf = (C.c_int * 64)()
    np_ = lib.fufft_plan_chains(n, VARIANT[variant], buf)
    if np_ < 0:
        raise FufftError(np_, "fufft_plan_chains")
    return list(buf[:np_])


def digit_order(n: int, variant: str = "auto") -> np.ndarray:
    perm = np.empty(n, dtype=np.int32)
    check(lib.fufft_digit_order(n, VARIANT[variant], perm.ctypes.data_as(C.POINTER(C.c_int32))),
          "fufft_digit_order")
    return perm


def plan_filter(x: np.ndarray, n: int, variant: str = "auto", layout: str = "dr",
                kind: int = FILTER_SPECTRUM, fold_inv_n: bool = True) -> np.ndarray:
    """Filter as the conv kernels read it, from a natural-order spectrum or taps."""
    src = np.ascontiguousarray(x, dtype=np.complex64).reshape(-1)
    if src.size != n:
        raise ValueError(f"plan_filter: {src.size} points given, n = {n}")
    out = np.empty(n, dtype=np.complex64)
    check(lib.fufft_plan_filter_f32(n, VARIANT[variant], LAYOUT[layout], kind, int(fold_inv_n),
                                    src.ctypes.data, out.ctypes.data), "fufft_plan_filter_f32")
    return out


TWIDDLES = {"accurate": 0, "reference": 1}


def twiddle_table_host(log_max: int, source: str = "accurate") -> np.ndarray:
    out = np.empty(2 << log_max, dtype=np.complex64)
    check(lib.fufft_twiddle_table_host_source(log_max, TWIDDLES[source], out.ctypes.data),
          "fufft_twiddle_table_host_source")
    return out


def set_twiddles(source: str, device: int = 0) -> None:
    """Base-twiddle source of the device table: "accurate" (default, fp64
    evaluated) or "reference" (the reference's fp32-angle cosf/sinf, with which
    the fp32 kernels reproduce its CPU transcription bit for bit)."""
    check(lib.fufft_set_twiddles(device, TWIDDLES[source]), "fufft_set_twiddles")


def get_twiddles(device: int = 0) -> str:
    v = C.c_int(-1)
    check(lib.fufft_get_twiddles(device, C.byref(v)), "fufft_get_twiddles")
    return {i: k for k, i in TWIDDLES.items()}[v.value]


# ---- launches ------------------------------------------------------------------------
# Each wrapper checks its tensors (_dev) against the sizes the call implies
# before the library sees them; the library then checks sizes, strides,
# enums and alignment again and returns a status, raised as FufftError.

def _mid(mid) -> int:
    """The C ABI id of a mid operation: a name of MID, or an id as it is (a
    policy added to the library's kernel sources has an id and no name here)."""
    if isinstance(mid, str):
        if mid not in MID:
            raise ValueError(f"mid must be one of {sorted(MID)} or a policy id, not {mid!r}")
        return MID[mid]
    return int(mid)


_MID_READS_FILTER = {MID["mul"]: True, MID["conj"]: True, MID["none"]: False}


def mid_reads_filter(mid) -> bool:
    """Whether the mid operation reads a filter: known here for the three
    named ones, asked of the library (fufft_mid_reads_filter) for any other
    id; FufftError for an id no policy of this build has."""
    m = _mid(mid)
    if m in _MID_READS_FILTER:
        return _MID_READS_FILTER[m]
    r = lib.fufft_mid_reads_filter(m)
    if r < 0:
        raise FufftError(r, "fufft_mid_reads_filter")
    return bool(r)


def _filt(filt, name: str, n: int, batch: int, stride: int, mid):
    """Spec of a filter (or spectrum) of n points per item and stride `stride`;
    None where the call does not read it (a mid operation that reads no
    filter, with no filter given)."""
    if filt is None and not mid_reads_filter(mid):
        return None
    return (filt, name, 8 * n * _count(stride, n, batch, name) if batch else 0, "complex")


def conv(inp, filt, out, n: int, batch: int, filt_stride: int = 0, mid: str = "mul",
         variant: str = "auto", layout: str = "dr", stream=None) -> None:
    nb = 8 * n * batch
    pi, pf, po = _ptrs((inp, "inp", nb, "complex"), _filt(filt, "filt", n, batch, filt_stride, mid),
                       (out, "out", nb, "complex"))
    check(lib.fufft_conv_f32(pi, pf, filt_stride, po, n, batch, _mid(mid), VARIANT[variant], LAYOUT[layout],
                             _stream(stream)), "fufft_conv_f32")


TIMER_STRIDE = 12
PHASES = ("load", "forward", "mid", "inverse", "store")


def transforms_per_workgroup(n: int, variant: str = "auto") -> int:
    k = lib.fufft_transforms_per_workgroup(n, VARIANT[variant])
    if k < 0:
        raise FufftError(k, "fufft_transforms_per_workgroup")
    return k


def conv_timed(inp, filt, out, timing, n: int, batch: int, timing_groups: int, filt_stride: int = 0,
               mid: str = "mul", variant: str = "auto", layout: str = "dr", stream=None) -> None:
    """fufft_conv_f32 with the in-kernel phase timer; timing is a device buffer
    of timing_groups * TIMER_STRIDE uint32 words (decode with decode_timing)."""
    nb = 8 * n * batch
    ts = (timing, "timing", 4 * TIMER_STRIDE * timing_groups, "words") if timing_groups else None
    pi, pf, po, pt = _ptrs((inp, "inp", nb, "complex"), _filt(filt, "filt", n, batch, filt_stride, mid),
                           (out, "out", nb, "complex"), ts)
    check(lib.fufft_conv_timed_f32(pi, pf, filt_stride, po, n, batch, _mid(mid), VARIANT[variant],
                                   LAYOUT[layout], pt, timing_groups, _stream(stream)),
          "fufft_conv_timed_f32")


def decode_timing(words: np.ndarray) -> dict:
    """Phase-timer records -> arrays: xcd, cu, se, start (cycles), and the cycles
    spent in each phase (differences of consecutive marks)."""
    w = np.asarray(words, dtype=np.uint32).reshape(-1, TIMER_STRIDE).astype(np.int64)
    marks = w[:, 6:11] & 0xFFFFFF
    phase_ids = w[:, 6:11] >> 24
    if not np.all(phase_ids == np.arange(1, 6)):
        raise ValueError("timer records carry unexpected phase ids")
    prev = np.concatenate([np.zeros((len(w), 1), np.int64), marks[:, :-1]], axis=1)
    return {
        "hw_id": w[:, 0], "xcd": w[:, 1] & 0xF, "cu": (w[:, 0] >> 8) & 0xF, "simd": (w[:, 0] >> 4) & 0x3,
        "realtime_ticks": w[:, 3], "start": w[:, 4] | (w[:, 5] << 32), "marks": marks,
        "phase_cycles": {name: marks[:, i] - prev[:, i] for i, name in enumerate(PHASES)},
        "total_cycles": marks[:, -1],
    }


def fwd(inp, spec, n: int, batch: int, variant: str = "auto", stream=None) -> None:
    nb = 8 * n * batch
    pi, ps = _ptrs((inp, "inp", nb, "complex"), (spec, "spec", nb, "complex"))
    check(lib.fufft_fwd_f32(pi, ps, n, batch, VARIANT[variant], _stream(stream)), "fufft_fwd_f32")


def apply(spec, filt, out, n: int, batch: int, spec_stride: int = 0, filt_stride: int = 0,
          mid: str = "mul", variant: str = "auto", layout: str = "dr", stream=None) -> None:
    ps, pf, po = _ptrs(_filt(spec, "spec", n, batch, spec_stride, "mul"),
                       _filt(filt, "filt", n, batch, filt_stride, mid), (out, "out", 8 * n * batch, "complex"))
    check(lib.fufft_apply_f32(ps, spec_stride, pf, filt_stride, po, n, batch, _mid(mid), VARIANT[variant],
                              LAYOUT[layout], _stream(stream)), "fufft_apply_f32")


def conv_r2(x, y, filt, u, v, n: int, batch: int, filt_stride: int = 0, variant: str = "auto",
            layout: str = "dr", stream=None) -> None:
    rb = 4 * n * batch
    px, py, pf, pu, pv = _ptrs((x, "x", rb, "real"), (y, "y", rb, "real"),
                               _filt(filt, "filt", n, batch, filt_stride, "mul"),
                               (u, "u", rb, "real"), (v, "v", rb, "real"))
    check(lib.fufft_conv_r2_f32(px, py, pf, filt_stride, pu, pv, n, batch, VARIANT[variant], LAYOUT[layout],
                                _stream(stream)), "fufft_conv_r2_f32")


def conv_bfp16(qin, ein, filt, qout, eout, n: int, batch: int, filt_stride: int = 0,
               mid: str = "mul", variant: str = "auto", layout: str = "dr", stream=None,
               block: int = BFP_BLOCK) -> None:
    """int16-BFP fused conv; one exponent per `block` points (64 .. n, a power of two)."""
    qb, eb = 4 * n * batch, (n * batch) // block if block > 0 else 0
    pq, pe, pf, pqo, peo = _ptrs((qin, "qin", qb, "bfp"), (ein, "ein", eb, "exp"),
                                 _filt(filt, "filt", n, batch, filt_stride, mid),
                                 (qout, "qout", qb, "bfp"), (eout, "eout", eb, "exp"))
    check(lib.fufft_conv_bfp16(pq, pe, pf, filt_stride, pqo, peo, n, batch, block, _mid(mid), VARIANT[variant],
                               LAYOUT[layout], _stream(stream)), "fufft_conv_bfp16")


def conv_bfp16_scaled(qin, sin, qfilt, sfilt, qout, sout, n: int, batch: int, filt_stride: int = 0,
                      mid: str = "mul", variant: str = "auto", layout: str = "dr", stream=None) -> None:
    """int16-BFP fused conv in the reference's own format (fufft_pipeline_v16_bfp):
    one fp32 scale per transform (sin / sout, batch floats), the filter as
    int16 pairs with one fp32 scale per filter, in the slots of the fp32
    filter's layout ("dr", the reference's digit order; "lane"; "bperm")."""
    qb = 4 * n * batch
    nf = _count(filt_stride, n, batch, "qfilt") if batch else 0
    reads = mid_reads_filter(mid)
    fq = None if (qfilt is None and not reads) else (qfilt, "qfilt", 4 * n * nf, "bfp")
    fs = None if (sfilt is None and not reads) else (sfilt, "sfilt", 4 * nf, "scale")
    pq, ps, pfq, pfs, pqo, pso = _ptrs((qin, "qin", qb, "bfp"), (sin, "sin", 4 * batch, "scale"), fq, fs,
                                       (qout, "qout", qb, "bfp"), (sout, "sout", 4 * batch, "scale"))
    check(lib.fufft_conv_bfp16_scaled(pq, ps, pfq, pfs, filt_stride, pqo, pso, n, batch, _mid(mid),
                                      VARIANT[variant], LAYOUT[layout], _stream(stream)),
          "fufft_conv_bfp16_scaled")


def c2c(inp, out, n: int, batch: int, direction: int = FORWARD, variant: str = "auto",
        stream=None) -> None:
    """Natural-order batched C2C: forward, or the unnormalised inverse."""
    nb = 8 * n * batch
    pi, po = _ptrs((inp, "inp", nb, "complex"), (out, "out", nb, "complex"))
    check(lib.fufft_c2c_f32(pi, po, n, batch, direction, VARIANT[variant], _stream(stream)), "fufft_c2c_f32")


def plan_filter_device(inp, out, n: int, count: int = 1, variant: str = "auto", layout: str = "dr",
                       kind: int = FILTER_SPECTRUM, fold_inv_n: bool = True, stream=None) -> None:
    """fufft_plan_filter_f32 on device memory, for count filters."""
    nb = 8 * n * count
    pi, po = _ptrs((inp, "inp", nb, "complex"), (out, "out", nb, "complex"))
    check(lib.fufft_plan_filter_device_f32(pi, po, n, count, VARIANT[variant], LAYOUT[layout], kind,
                                           int(fold_inv_n), _stream(stream)),
          "fufft_plan_filter_device_f32")


def plan_filter_large_device(inp, out, n: int, count: int = 1, kind: int = FILTER_SPECTRUM,
                             fold_inv_n: bool = True, variant: str = "auto", stream=None) -> None:
    nb = 8 * n * count
    pi, po = _ptrs((inp, "inp", nb, "complex"), (out, "out", nb, "complex"))
    check(lib.fufft_plan_filter_large_device_f32(pi, po, n, count, VARIANT[variant], kind, int(fold_inv_n),
                                                 _stream(stream)),
          "fufft_plan_filter_large_device_f32")


def plan_filter2d_device(inp, out, h: int, w: int, count: int = 1, kind: int = FILTER_SPECTRUM,
                         fold_inv_n: bool = True, layout: str = "dr", stream=None) -> None:
    nb = 8 * h * w * count
    pi, po = _ptrs((inp, "inp", nb, "complex"), (out, "out", nb, "complex"))
    check(lib.fufft_plan_filter2d_device_f32(pi, po, h, w, count, LAYOUT[layout], kind, int(fold_inv_n),
                                             _stream(stream)),
          "fufft_plan_filter2d_device_f32")


# ---- four-step large N -------------------------------------------------------------------

def large_plan(n: int) -> tuple[int, int]:
    """(lout, mid): n = 16^lout * mid, the middle a single-launch size."""
    lout, mid = C.c_int(), C.c_int()
    check(lib.fufft_large_plan(n, C.byref(lout), C.byref(mid)), "fufft_large_plan")
    return lout.value, mid.value


def large_middle(variant: str = "auto") -> int:
    """Values per lane of the four-step middle a variant names: "v16" and
    "auto" the reference's radix-16 middle, "r8" the radix-8 one."""
    return 8 if variant == "r8" else 16


def large_digit_order(n: int, variant: str = "auto") -> np.ndarray:
    """Slot -> bin of the chained four-step order: [16]^lout, then the
    middle's radices ("v16"/"auto": run_large's order, bench_fufft.cu:410-428)."""
    perm = np.empty(n, dtype=np.int32)
    check(lib.fufft_large_digit_order(n, VARIANT[variant], perm.ctypes.data_as(C.POINTER(C.c_int32))),
          "fufft_large_digit_order")
    return perm


def plan_filter_large(x: np.ndarray, n: int, kind: int = FILTER_SPECTRUM,
                      fold_inv_n: bool = True, variant: str = "auto") -> np.ndarray:
    src = np.ascontiguousarray(x, dtype=np.complex64).reshape(-1)
    if src.size != n:
        raise ValueError(f"plan_filter_large: {src.size} points given, n = {n}")
    out = np.empty(n, dtype=np.complex64)
    check(lib.fufft_plan_filter_large_f32(n, VARIANT[variant], kind, int(fold_inv_n), src.ctypes.data,
                                          out.ctypes.data),
          "fufft_plan_filter_large_f32")
    return out


def conv_large(buf, filt, n: int, batch: int, filt_stride: int = 0, mid: str = "mul",
               variant: str = "auto", stream=None) -> None:
    """Four-step conv of a batch of n-point signals, in place on buf; the
    filter in the chain order of the same variant (large_digit_order)."""
    pb, pf = _ptrs((buf, "buf", 8 * n * batch, "complex"), _filt(filt, "filt", n, batch, filt_stride, mid))
    check(lib.fufft_conv_large_f32(pb, pf, filt_stride, n, batch, _mid(mid), VARIANT[variant], _stream(stream)),
          "fufft_conv_large_f32")


# ---- 2D ------------------------------------------------------------------------------------
# 2D filters carry a column order (layout): "dr" is the reference's,
# entry (r, c) = bin (rev_h(r), rev_w(c)); "lane" is this library's faster
# order, entry (r, c) = bin (rev_h(r), rev_w(slot(c))), slot = column_order2d.
# The planners and the launches default to "dr", so filters planned for the
# reference work unchanged; plan and launch with layout="lane" for speed.

def plan2d(h: int, w: int) -> tuple[int, int]:
    """(values per lane of the row plan, of the column plan)."""
    vr, vc = C.c_int(), C.c_int()
    check(lib.fufft_plan2d(h, w, C.byref(vr), C.byref(vc)), "fufft_plan2d")
    return vr.value, vc.value


def column_order2d(h: int, w: int) -> np.ndarray:
    """slot[c]: the row plan's digit-order slot held by column c of "lane" 2D filters and spectra."""
    out = np.empty(w, dtype=np.int32)
    check(lib.fufft_plan2d_column_order(h, w, out.ctypes.data_as(C.POINTER(C.c_int32))),
          "fufft_plan2d_column_order")
    return out


def plan_filter2d(x: np.ndarray, h: int, w: int, kind: int = FILTER_SPECTRUM,
                  fold_inv_n: bool = True, layout: str = "dr") -> np.ndarray:
    """2D filter as the column kernels read it in `layout`."""
    src = np.ascontiguousarray(x, dtype=np.complex64).reshape(-1)
    if src.size != h * w:
        raise ValueError(f"plan_filter2d: {src.size} points given, h * w = {h * w}")
    out = np.empty(h * w, dtype=np.complex64)
    check(lib.fufft_plan_filter2d_f32(h, w, LAYOUT[layout], kind, int(fold_inv_n), src.ctypes.data,
                                      out.ctypes.data), "fufft_plan_filter2d_f32")
    return out


def conv2d(inp, filt, out, h: int, w: int, batch: int, filt_stride: int = 0, mid: str = "mul",
           layout: str = "dr", stream=None) -> None:
    nb = 8 * h * w * batch
    pi, pf, po = _ptrs((inp, "inp", nb, "complex"), _filt(filt, "filt", h * w, batch, filt_stride, mid),
                       (out, "out", nb, "complex"))
    check(lib.fufft_conv2d_f32(pi, pf, filt_stride, po, h, w, batch, _mid(mid), LAYOUT[layout],
                               _stream(stream)), "fufft_conv2d_f32")


def conv2d_r2(x, y, filt, u, v, work, h: int, w: int, batch: int, filt_stride: int = 0,
              layout: str = "dr", stream=None) -> None:
    rb = 4 * h * w * batch
    px, py, pf, pu, pv, pw = _ptrs((x, "x", rb, "real"), (y, "y", rb, "real"),
                                   _filt(filt, "filt", h * w, batch, filt_stride, "mul"),
                                   (u, "u", rb, "real"), (v, "v", rb, "real"), (work, "work", 2 * rb, "complex"))
    check(lib.fufft_conv2d_r2_f32(px, py, pf, filt_stride, pu, pv, pw, h, w, batch, LAYOUT[layout],
                                  _stream(stream)), "fufft_conv2d_r2_f32")


def conv2d_r2_noalloc(x, y, filt, u, v, h: int, w: int, batch: int, filt_stride: int = 0,
                      layout: str = "dr", stream=None) -> None:
    """conv2d_r2 without a workspace: the library's static scratch holds the
    packed images (SCRATCH_BYTES per GPU; calls that overlap on one GPU race)."""
    rb = 4 * h * w * batch
    px, py, pf, pu, pv = _ptrs((x, "x", rb, "real"), (y, "y", rb, "real"),
                               _filt(filt, "filt", h * w, batch, filt_stride, "mul"),
                               (u, "u", rb, "real"), (v, "v", rb, "real"))
    check(lib.fufft_conv2d_r2_noalloc_f32(px, py, pf, filt_stride, pu, pv, h, w, batch, LAYOUT[layout],
                                          _stream(stream)), "fufft_conv2d_r2_noalloc_f32")


def fwd2d(inp, spec, h: int, w: int, batch: int, stream=None) -> None:
    nb = 8 * h * w * batch
    pi, ps = _ptrs((inp, "inp", nb, "complex"), (spec, "spec", nb, "complex"))
    check(lib.fufft_fwd2d_f32(pi, ps, h, w, batch, _stream(stream)), "fufft_fwd2d_f32")


def apply2d(spec, filt, out, h: int, w: int, batch: int, spec_stride: int = 0, filt_stride: int = 0,
            mid: str = "mul", layout: str = "dr", stream=None) -> None:
    np_ = h * w
    ps, pf, po = _ptrs(_filt(spec, "spec", np_, batch, spec_stride, "mul"),
                       _filt(filt, "filt", np_, batch, filt_stride, mid), (out, "out", 8 * np_ * batch, "complex"))
    check(lib.fufft_apply2d_f32(ps, spec_stride, pf, filt_stride, po, h, w, batch, _mid(mid), LAYOUT[layout],
                                _stream(stream)), "fufft_apply2d_f32")


def stream_copy(inp, out, nbytes: int, nontemporal: bool = False, stream=None) -> None:
    """HBM stream ceiling: copy nbytes with the conv kernels' buffer instructions."""
    pi, po = _ptrs((inp, "inp", nbytes, "complex"), (out, "out", nbytes, "complex"))
    check(lib.fufft_stream_f32(pi, po, nbytes, int(nontemporal), _stream(stream)), "fufft_stream_f32")


def stream_copy_shape(inp, out, nbytes: int, loads: int = 8, per: int = 1, groups: int = 0,
                      load_policy: int = 0, store_policy: int = 0, width: int = 16, lanes: int = 256,
                      stream=None) -> None:
    """The stream copy in a chosen shape (fufft_stream_shape_f32): workgroups
    of `lanes` lanes, `loads` loads of `width` bytes per lane in flight, `per`
    consecutive tiles per workgroup or a persistent grid of `groups`
    workgroups, cache policies SC0 = 1, NT = 2."""
    pi, po = _ptrs((inp, "inp", nbytes, "complex"), (out, "out", nbytes, "complex"))
    check(lib.fufft_stream_shape_f32(pi, po, nbytes, lanes, width, loads, per, groups, load_policy, store_policy,
                                     _stream(stream)), "fufft_stream_shape_f32")


def bfp_exponent(absmax: float) -> int:
    return lib.fufft_bfp_exponent(absmax)


def bfp_quantize(x: np.ndarray, block: int = BFP_BLOCK) -> tuple[np.ndarray, np.ndarray]:
    src = np.ascontiguousarray(x, dtype=np.complex64).reshape(-1)
    q = np.empty(2 * src.size, dtype=np.int16)
    e = np.empty(max(src.size // block, 1), dtype=np.int8)
    check(lib.fufft_bfp_quantize(src.ctypes.data, src.size, block, q.ctypes.data, e.ctypes.data),
          "fufft_bfp_quantize")
    return q, e[: src.size // block]


def bfp_scaled_quantize(x: np.ndarray, n: int) -> tuple[np.ndarray, np.ndarray]:
    """The reference's codec (fufft_bfp_scaled_quantize): int16 pairs and one
    fp32 scale per transform of n points."""
    src = np.ascontiguousarray(x, dtype=np.complex64).reshape(-1)
    if src.size % n:
        raise ValueError(f"{src.size} points are not whole transforms of {n}")
    q = np.empty(2 * src.size, dtype=np.int16)
    sc = np.empty(max(src.size // n, 1), dtype=np.float32)
    check(lib.fufft_bfp_scaled_quantize(src.ctypes.data, n, src.size // n, q.ctypes.data, sc.ctypes.data),
          "fufft_bfp_scaled_quantize")
    return q, sc[: src.size // n]


def _int16_words(q) -> np.ndarray:
    """BFP words as a contiguous int16 array; any other dtype is refused (an
    int32 array would otherwise be read as pairs of int16)."""
    q = np.asarray(q)
    if q.dtype != np.int16:
        raise TypeError(f"BFP words must be int16, got {q.dtype}")
    return np.ascontiguousarray(q).reshape(-1)


def bfp_scaled_dequantize(q: np.ndarray, scale: np.ndarray, n: int) -> np.ndarray:
    q = _int16_words(q)
    if n < 1 or q.size % (2 * n):
        raise ValueError(f"{q.size} int16 words are not whole transforms of {n} points")
    count = q.size // (2 * n)
    sc = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    if sc.size < count:
        raise ValueError(f"{count} transforms need {count} scales, {sc.size} given")
    x = np.empty(count * n, dtype=np.complex64)
    check(lib.fufft_bfp_scaled_dequantize(q.ctypes.data, sc.ctypes.data, n, count, x.ctypes.data),
          "fufft_bfp_scaled_dequantize")
    return x


def bfp_dequantize(q: np.ndarray, e: np.ndarray, block: int = BFP_BLOCK) -> np.ndarray:
    q = _int16_words(q)
    npts = q.size // 2
    if q.size % 2 or block < 1 or npts % block:
        raise ValueError(f"{q.size} int16 words are not whole blocks of {block} points")
    ex = np.asarray(e)
    if ex.dtype != np.int8:
        raise TypeError(f"BFP exponents must be int8, got {ex.dtype}")
    ex = np.ascontiguousarray(ex).reshape(-1)
    if ex.size < npts // block:
        raise ValueError(f"{npts // block} blocks need {npts // block} exponents, {ex.size} given")
    x = np.empty(npts, dtype=np.complex64)
    check(lib.fufft_bfp_dequantize(q.ctypes.data, ex.ctypes.data, npts, block, x.ctypes.data),
          "fufft_bfp_dequantize")
    return x
