"""Write the golden fixtures from the reference's compiled CPU transcription.

Run in the build container, where /root/reference exists and `make -C oracle
ref` has built oracle/_ref/libfufft_ref.so:

    python -m tests.golden.make_golden              # every fixture
    python -m tests.golden.make_golden bfp_scaled   # only bfp_scaled_n*.npz
    python -m tests.golden.make_golden fourstep_v16 # only fourstep_n32768_mid2048_v16.npz
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O
from tests.golden.golden import HERE


def _cu(rng, shape):
    return (rng.uniform(-1, 1, shape) + 1j * rng.uniform(-1, 1, shape)).astype(np.complex64)


def _lead_count(n, v):
    rads = O.factor(n, v)
    return (rads[0] if rads[0] != v else 1), rads.count(v)


def _save(name, **kw):
    np.savez_compressed(HERE / f"{name}.npz", **kw)


def bfp_scaled(R) -> None:
    """The reference's own BFP format (kernel_v16_bfp, verify_kernel.cpp:1107-1135):
    int16 pairs and one fp32 scale per transform in and out, a shared int16
    filter with one scale, at the sizes of BASELINE config 3."""
    rng = np.random.default_rng(20261203)
    for n in (512, 4096):
        batch = 4
        x = (rng.standard_normal((batch, n)) + 1j * rng.standard_normal((batch, n))).astype(np.complex64)
        x = (x * (10.0 ** rng.uniform(-3, 3, (batch, 1)))).astype(np.complex64)
        aq, asc = np.empty(2 * n * batch, np.int16), np.empty(batch, np.float32)
        for t in range(batch):
            xt = np.ascontiguousarray(x[t])
            asc[t] = R.ref_vk_bfp_quantize(xt.ctypes.data, n, aq[2 * n * t:].ctypes.data)
        b = _cu(rng, (1, n))[0] / n
        bdr = np.ascontiguousarray(b[O.mixedrev(O.kernel_plan(n, 16))])
        bq = np.empty(2 * n, np.int16)
        bsc = np.float32(R.ref_vk_bfp_quantize(bdr.ctypes.data, n, bq.ctypes.data))
        lead, nrv = _lead_count(n, 16)
        oq, osc = np.empty_like(aq), np.empty(batch, np.float32)
        R.ref_vk_v16_bfp(n, lead, nrv, aq.ctypes.data, asc.ctypes.data, bq.ctypes.data, float(bsc),
                         oq.ctypes.data, osc.ctypes.data, batch)
        _save(f"bfp_scaled_n{n}", kind="bfp_scaled", n=n, aq=aq, asc=asc, bq=bq, bsc=np.array([bsc]),
              oq=oq, osc=osc)


def fourstep_v16(R) -> None:
    """The reference bench's own four-step configuration,
    run_large<32768, 1, 16, 2048, 8, 2> (bench_fufft.cu:519): one radix-16
    outer level around the V=16 middle (lead 8, two radix-16 passes), the
    filter in run_large's chain order (bench_fufft.cu:410-428), computed by
    the reference's transcription conv_foursteps_cfg with the V=16 middle
    (verify_kernel.cpp:373-394)."""
    rng = np.random.default_rng(20261204)
    n, mid = 32768, 2048
    a, b = _cu(rng, (1, n)), _cu(rng, (1, n)) / n
    bdr = np.ascontiguousarray(b[:, O.mixedrev(O.large_plan(1, mid, 16, ref=True))])
    A = a.copy()
    R.ref_vk_conv_foursteps_cfg(A.ctypes.data, bdr.ctypes.data, n, 1, 16, mid, 1)
    _save("fourstep_n32768_mid2048_v16", kind="fourstep", n=n, lout=1, mid=mid, mid_v=16, a=a, bdr=bdr,
          out=A.reshape(-1))


def main() -> None:
    R = O.load_ref()
    if R is None:
        raise SystemExit("oracle/_ref/libfufft_ref.so is not built (needs /root/reference)")
    rng = np.random.default_rng(20261201)
    save = _save

    for n in (64, 512, 1024):
        batch = 2
        a, b = _cu(rng, (batch, n)), _cu(rng, (batch, n)) / n
        bdr = np.ascontiguousarray(b[:, O.mixedrev(O.kernel_plan(n, 16))])
        lead, nrv = _lead_count(n, 16)
        out = np.empty_like(a)
        R.ref_vk_pipeline_v16(n, lead, nrv, 1, a.ctypes.data, bdr.ctypes.data, out.ctypes.data, batch)
        save(f"v16_n{n}", kind="v16", n=n, a=a, bdr=bdr, out=out.reshape(-1))

    for n in (512, 4096):
        batch = 1
        a, b = _cu(rng, (batch, n)), _cu(rng, (batch, n)) / n
        bdr = np.ascontiguousarray(b[:, O.mixedrev(O.kernel_plan(n, 8))])
        lead, nr8 = _lead_count(n, 8)
        out = np.empty_like(a)
        R.ref_vk_pipeline_ip(n, lead, nr8, 1, a.ctypes.data, bdr.ctypes.data, out.ctypes.data, batch)
        save(f"r8_n{n}", kind="r8", n=n, a=a, bdr=bdr, out=out.reshape(-1))

    n, batch = 512, 2
    a, b = _cu(rng, (batch, n)), _cu(rng, (batch, n)) / n
    bdr = np.ascontiguousarray(b[:, O.mixedrev(O.kernel_plan(n, 8))])
    lead, nr8 = _lead_count(n, 8)
    spec, out = np.empty_like(a), np.empty_like(a)
    R.ref_vk_pipeline_fwd(n, lead, nr8, 1, a.ctypes.data, spec.ctypes.data, batch)
    R.ref_vk_pipeline_apply(n, lead, nr8, 1, spec.ctypes.data, bdr.ctypes.data, out.ctypes.data, batch)
    save("split_n512", kind="split", n=n, a=a, bdr=bdr, spec=spec.reshape(-1), out=out.reshape(-1))

    h, w = 64, 64
    a, b = _cu(rng, (1, h, w)), _cu(rng, (1, h, w)) / (h * w)
    bdr = np.ascontiguousarray(b[:, O.mixedrev(O.kernel_plan(h, 8))][:, :, O.mixedrev(O.kernel_plan(w, 8))])
    out = np.empty_like(a)
    R.ref_vk_conv2d(h, w, a.ctypes.data, bdr.ctypes.data, out.ctypes.data, 1)
    save("conv2d_64x64", kind="conv2d", h=h, w=w, a=a, bdr=bdr, out=out.reshape(-1))

    n, batch = 256, 2
    x = rng.uniform(-1, 1, (batch, n)).astype(np.float32)
    y = rng.uniform(-1, 1, (batch, n)).astype(np.float32)
    b = _cu(rng, (batch, n)) / n
    bdr = np.ascontiguousarray(b[:, O.mixedrev(O.kernel_plan(n, 8))])
    lead, nr8 = _lead_count(n, 8)
    u, v = np.empty_like(x), np.empty_like(y)
    R.ref_vk_conv_r2(n, lead, nr8, 1, x.ctypes.data, y.ctypes.data, bdr.ctypes.data,
                     u.ctypes.data, v.ctypes.data, batch)
    save("r2_n256", kind="r2", n=n, x=x, y=y, bdr=bdr, u=u.reshape(-1), v=v.reshape(-1))

    n, mid = 4096, 256
    a, b = _cu(rng, (1, n)), _cu(rng, (1, n)) / n
    bdr = np.ascontiguousarray(b[:, O.mixedrev(O.large_plan(1, mid))])
    A = a.copy()
    R.ref_vk_conv_foursteps_cfg(A.ctypes.data, bdr.ctypes.data, n, 1, 16, mid, 1)
    save("fourstep_n4096_mid256", kind="fourstep", n=n, lout=1, mid=mid, a=a, bdr=bdr, out=A.reshape(-1))

    # drawn last so the fixtures above keep their inputs
    n, batch = 512, 2
    a = _cu(rng, (batch, n))
    out = np.empty_like(a)
    R.ref_vk_c2c(n, 1, a.ctypes.data, out.ctypes.data, batch)
    save("c2c_stockham_n512", kind="c2c_stockham", n=n, a=a, out=out.reshape(-1))

    # Fixtures at sizes the GPU kernels run with the reference's own plans, so
    # the GPU tests can compare against the reference directly (in
    # reference-twiddle mode).  A second generator keeps the inputs above.
    rng = np.random.default_rng(20261202)
    for n in (1024, 2048):                       # radix-8 with a lead 2 / 4 pass
        a, b = _cu(rng, (1, n)), _cu(rng, (1, n)) / n
        bdr = np.ascontiguousarray(b[:, O.mixedrev(O.kernel_plan(n, 8))])
        lead, nr8 = _lead_count(n, 8)
        out = np.empty_like(a)
        R.ref_vk_pipeline_ip(n, lead, nr8, 1, a.ctypes.data, bdr.ctypes.data, out.ctypes.data, 1)
        save(f"r8_n{n}", kind="r8", n=n, a=a, bdr=bdr, out=out.reshape(-1))

    for n in (2048, 4096):                       # radix 16 with a lead 8 pass / pure 16^3
        a, b = _cu(rng, (1, n)), _cu(rng, (1, n)) / n
        bdr = np.ascontiguousarray(b[:, O.mixedrev(O.kernel_plan(n, 16))])
        lead, nrv = _lead_count(n, 16)
        out = np.empty_like(a)
        R.ref_vk_pipeline_v16(n, lead, nrv, 1, a.ctypes.data, bdr.ctypes.data, out.ctypes.data, 1)
        save(f"v16_n{n}", kind="v16", n=n, a=a, bdr=bdr, out=out.reshape(-1))

    n, batch = 512, 2                            # two-for-one real, radix 8
    x = rng.uniform(-1, 1, (batch, n)).astype(np.float32)
    y = rng.uniform(-1, 1, (batch, n)).astype(np.float32)
    b = _cu(rng, (batch, n)) / n
    bdr = np.ascontiguousarray(b[:, O.mixedrev(O.kernel_plan(n, 8))])
    lead, nr8 = _lead_count(n, 8)
    u, v = np.empty_like(x), np.empty_like(y)
    R.ref_vk_conv_r2(n, lead, nr8, 1, x.ctypes.data, y.ctypes.data, bdr.ctypes.data,
                     u.ctypes.data, v.ctypes.data, batch)
    save("r2_n512", kind="r2", n=n, x=x, y=y, bdr=bdr, u=u.reshape(-1), v=v.reshape(-1))

    n, mid = 8192, 512                           # four-step, radix-8 middle (the GPU's plan)
    a, b = _cu(rng, (1, n)), _cu(rng, (1, n)) / n
    bdr = np.ascontiguousarray(b[:, O.mixedrev(O.large_plan(1, mid, 8))])
    A = a.copy()
    R.ref_vk_conv_foursteps_cfg(A.ctypes.data, bdr.ctypes.data, n, 1, 16, mid, 0)
    save("fourstep_n8192_mid512_r8", kind="fourstep", n=n, lout=1, mid=mid, mid_v=8, a=a, bdr=bdr,
         out=A.reshape(-1))

    bfp_scaled(R)
    fourstep_v16(R)


if __name__ == "__main__":
    import sys
    parts = {"bfp_scaled": bfp_scaled, "fourstep_v16": fourstep_v16}
    if sys.argv[1:] and sys.argv[1] in parts:    # only one group of fixtures
        ref = O.load_ref()
        if ref is None:
            raise SystemExit("oracle/_ref/libfufft_ref.so is not built (needs /root/reference)")
        parts[sys.argv[1]](ref)
    else:
        main()
