/*
 * fuFFT-for-MI355X CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker, never the product: only tests/, the smoke()
 * entry and bench.py's cpu_baseline leg may load it.  The HIP library must
 * never route through it.
 *
 * It restates, in plain C, the reference's CPU algorithm for the fused
 * cyclic-convolution path (in-place DIF -> pointwise mid operation -> in-place
 * DIT, mixed radix, digit order never materialised):
 *   - radix-2/4/8/16 butterflies and their algebraic specialisations
 *     (reference fufft.cuh:208-450, 504-547, 652-689; transcribed on the CPU in
 *     verify_kernel.cpp:31-86, 1000-1011, 1100-1120)
 *   - stage twiddles by recurrence: one base twiddle W^j per group, the rest
 *     by repeated complex multiplication, single chain (fufft.cuh:436-450) or
 *     the radix-16 even/odd chains (fufft.cuh:701-720)
 *   - the in-place radix-R pass over groups (b, j) with taps b*R*M + j + k*M
 *     (fufft.cuh:722-756, 1113-1140; cpu_mixed.cpp:116-153)
 *   - factorisation lead * V^k with the leftover radix first
 *     (cpu_mixed.cpp:36-49) and the bit-group reversal that a DIF leaves
 *     behind (cpu_mixed.cpp:176-192, verify_kernel.cpp:460-477)
 *   - the Mid policies multiply / conjugate-multiply / nothing
 *     (fufft.cuh:616-650)
 *   - four-step = monolithic chain with outer radix passes first
 *     (verify_kernel.cpp:378-432), 2D rows-then-columns (verify_kernel.cpp:
 *     681-722), two-for-one real packing (verify_kernel.cpp:580-615), split
 *     forward / apply (verify_kernel.cpp:794-836)
 *   - the fp64 mixed-radix CPU conv path with per-twiddle cos/sin
 *     (cpu_mixed.cpp:116-174), used as the timed CPU baseline
 *
 * Twiddle source.  The reference computes W^j = (cosf, sinf)(step*j) with
 * step = SIGN*2pi/(R*M) in float (verify_kernel.cpp:31, fufft.cuh:362-371).
 * OR_TW_LIBM reproduces exactly that; OR_TW_TABLE takes W^j from the
 * correctly-rounded table (float)cos/sin(2*pi*j/P) computed in double, which
 * is what the HIP kernels read.  Every other operation is identical in the two
 * modes, and all arithmetic uses the same operation order and explicit fmaf
 * as the reference, so with OR_TW_LIBM the oracle is bit-identical to the
 * reference's own CPU transcription and with OR_TW_TABLE it is bit-identical
 * to the HIP kernels.
 *
 * Block floating point: the reference stores int16 with one fp32 scale per
 * transform (fufft.cuh:1572-1612).  This build stores int16 pairs with one
 * int8 exponent per block of contiguous points; the exponent rule is this
 * build's own and is pinned by closed-form boundary tests (or_bfp_exponent).
 *
 * Complex data is interleaved float (re, im) or double (re, im).
 */
#ifndef FUFFT_ORACLE_H
#define FUFFT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_TW_LIBM = 0, OR_TW_TABLE = 1 };
/* how the R-1 stage twiddles of a group are generated from W^j */
enum { OR_CHAIN_SINGLE = 0,   /* w, w*w1, w*w1*w1 ... (fufft.cuh:436-450)   */
       OR_CHAIN_EVENODD = 1,  /* radix 16 only: even/odd chains (701-720)  */
       OR_CHAIN_DIRECT = 2 }; /* every W^(jk) straight from the table       */
enum { OR_MID_MUL = 0, OR_MID_CONJ = 1, OR_MID_NONE = 2 };

#define OR_MAX_PASSES 32

/* n = lead * v^k, lead < v placed first; returns the pass count, 0 if n is
 * not a power of two >= 2.  (cpu_mixed.cpp:36-49) */
int or_factor(int n, int v, int* radices);

/* slot idx of a DIF output holds bin or_mixedrev(idx): the bit groups of
 * widths log2(radix) in pass order, read MSB-first and emitted reversed.
 * (cpu_mixed.cpp:176-192; verify_kernel.cpp:460-477) */
int or_mixedrev(int idx, const int* radices, int np);

/* base twiddle (cos, sin)(SIGN * 2*pi*j/P) from the selected source */
void or_twiddle(int twmode, int sign, int P, int j, float* c, float* s);

/* one in-place radix-R pass over len complex points (len % (R*M) == 0);
 * dit = 0: butterfly then twiddle, dit = 1: twiddle then butterfly */
void or_pass_f32(float* buf, int64_t len, int R, int M, int sign, int dit,
                 int chain, int twmode);

/* fused conv of batch signals of n points: DIF over radices (pass order),
 * mid with filt (digit order, signal t uses filt + 2*(t*filt_stride)),
 * DIT in reverse pass order.  in may equal out. */
void or_conv_f32(const float* in, const float* filt, int64_t filt_stride,
                 float* out, int n, int64_t batch,
                 const int* radices, const int* chains, int np,
                 int mid, int twmode);

/* split path: forward DIF only (natural -> digit order spectrum) */
void or_fwd_f32(const float* in, float* spec, int n, int64_t batch,
                const int* radices, const int* chains, int np, int twmode);

/* split path: spec (+ spec_stride per signal, 0 = broadcast) mid filt, then
 * DIT -> natural order out */
void or_apply_f32(const float* spec, int64_t spec_stride,
                  const float* filt, int64_t filt_stride, float* out,
                  int n, int64_t batch, const int* radices, const int* chains,
                  int np, int mid, int twmode);

/* two real signals per complex transform, real filter (fufft.cuh:1260-1330) */
void or_conv_r2_f32(const float* x, const float* y, const float* filt,
                    int64_t filt_stride, float* u, float* v, int n,
                    int64_t batch, const int* radices, const int* chains,
                    int np, int twmode);

/* natural-order C2C: sign -1 forward DIF then slot s -> bin mixedrev(s);
 * sign +1 bin mixedrev(s) -> slot s then DIT, unnormalised.  in may equal out.
 * (fufft_c2c, fufft.cuh:879-904, is the forward Stockham counterpart) */
void or_c2c_f32(const float* in, float* out, int n, int64_t batch,
                const int* radices, const int* chains, int np, int sign,
                int twmode);

/* 2D conv of h x w images (row-major): row DIF, column DIF, mid, column DIT,
 * row DIT (verify_kernel.cpp:700-722).  filt slot (r, c) holds spectrum bin
 * (mixedrev_h(r), mixedrev_w(c)). */
void or_conv2d_f32(const float* in, const float* filt, int64_t filt_stride,
                   float* out, int h, int w, int64_t batch,
                   const int* rad_h, const int* ch_h, int nph,
                   const int* rad_w, const int* ch_w, int npw,
                   int mid, int twmode);

/* 2D split path: rows DIF then columns DIF, spectrum in 2D digit order */
void or_fwd2d_f32(const float* in, float* spec, int h, int w, int64_t batch,
                  const int* rad_h, const int* ch_h, int nph,
                  const int* rad_w, const int* ch_w, int npw, int twmode);
void or_apply2d_f32(const float* spec, int64_t spec_stride, const float* filt,
                    int64_t filt_stride, float* out, int h, int w,
                    int64_t batch, const int* rad_h, const int* ch_h, int nph,
                    const int* rad_w, const int* ch_w, int npw, int mid,
                    int twmode);

/* ---- block floating point (this build's rule) ---------------------------
 * exponent e of a block with abs-max a (over |re| and |im|):
 *   a == 0 or a subnormal          -> e = -128
 *   otherwise the smallest integer with a <= 32767 * 2^e, clamped to >= -128
 * q = rint(x * 2^-e) (round half to even), |q| <= 32767 by construction;
 * x' = q * 2^e.  A point is two int16 (re low halfword, im high halfword). */
int  or_bfp_exponent(float absmax);
void or_bfp_quantize(const float* x, int64_t npts, int block,
                     int16_t* q, int8_t* e);
void or_bfp_dequantize(const int16_t* q, const int8_t* e, int64_t npts,
                       int block, float* x);
void or_bfp_conv(const int16_t* qin, const int8_t* ein, const float* filt,
                 int64_t filt_stride, int16_t* qout, int8_t* eout, int n,
                 int64_t batch, int block, const int* radices,
                 const int* chains, int np, int mid, int twmode);

/* ---- fp64 references ------------------------------------------------------ */
/* iterative radix-2 FFT, natural order in and out, unnormalised
 * (an algorithm independent of the mixed-radix path; verify_kernel.cpp:434) */
void or_fft2_f64(double* x, int n, int sign);
/* fp64 truth for the conv: out = IDFT(DFT(a) mid spec), spec in natural
 * order with 1/N already folded in, spec_stride 0 = shared */
void or_conv_spec_f64(const float* a, const float* spec, int64_t spec_stride,
                      double* out, int n, int64_t batch, int mid);
/* restated cpu_mixed fp64 conv path: DIF with per-twiddle cos/sin, multiply
 * by a digit-ordered spectrum, DIT (cpu_mixed.cpp:116-174, 252-267) */
void or_mixed_conv_f64(const double* a, const double* spec_dr, double* out,
                       int n, int64_t batch, int v);

double or_rel_l2_f32(const float* x, const float* y, int64_t ncomplex);
double or_rel_l2_f32_f64(const float* x, const double* y, int64_t ncomplex);

#ifdef __cplusplus
}
#endif
#endif
