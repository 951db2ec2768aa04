/*
 * fuFFT-for-MI355X CPU oracle -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Plain C99.  Build with -ffp-contract=off: the operation order below is the
 * contract, and a contracted a*b+c would break bit-identity with both the
 * reference's CPU transcription and the HIP kernels.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct { float x, y; } c32;
typedef struct { double x, y; } c64;

/* constants as spelled in fufft.cuh:40 and 517-518 */
static const float R2  = 0.70710678118654752440f;
static const float C16 = 0.92387953251128673848f;
static const float S16 = 0.38268343236508977173f;

static inline c32 mk(float x, float y) { c32 r; r.x = x; r.y = y; return r; }
static inline c32 cadd(c32 a, c32 b) { return mk(a.x + b.x, a.y + b.y); }
static inline c32 csub(c32 a, c32 b) { return mk(a.x - b.x, a.y - b.y); }

/* fufft.cuh:236-260 (C++ form): 2 MUL + 2 FMA */
static inline c32 cmul(c32 a, c32 b)
{
   return mk(fmaf(a.x, b.x, -a.y * b.y), fmaf(a.x, b.y, a.y * b.x));
}

/* x (+-i): swap and negate (fufft.cuh:263-287) */
static inline c32 cmul_i(c32 a, int sign)
{
   return sign < 0 ? mk(a.y, -a.x) : mk(-a.y, a.x);
}

/* x w8^1 = r2 (1, sign): 2 add + 2 mul (fufft.cuh:289-320) */
static inline c32 cmul_w1(c32 a, int sign)
{
   return sign < 0 ? mk(R2 * (a.x + a.y), R2 * (a.y - a.x))
                   : mk(R2 * (a.x - a.y), R2 * (a.x + a.y));
}

/* x w8^3 = r2 (-1, sign) (fufft.cuh:322-355) */
static inline c32 cmul_w3(c32 a, int sign)
{
   return sign < 0 ? mk(R2 * (a.y - a.x), R2 * (-a.x - a.y))
                   : mk(R2 * (-a.x - a.y), R2 * (a.x - a.y));
}

/* x W16^k (fufft.cuh:521-535) */
static inline c32 mul_w16(int k, c32 x, int sign)
{
   const float s = (float)sign;
   switch(k) {
      case 0:  return x;
      case 1:  return cmul(x, mk( C16, s * S16));
      case 2:  return cmul_w1(x, sign);
      case 3:  return cmul(x, mk( S16, s * C16));
      case 4:  return cmul_i(x, sign);
      case 5:  return cmul(x, mk(-S16, s * C16));
      case 6:  return cmul_w3(x, sign);
      default: return cmul(x, mk(-C16, s * S16));
   }
}

/* radix-8 in three radix-2 stages, natural-order output (fufft.cuh:377-405) */
static void dft8(const c32* u, c32* v, int sign)
{
   const c32 a0 = cadd(u[0], u[4]);
   const c32 a1 = cadd(u[1], u[5]);
   const c32 a2 = cadd(u[2], u[6]);
   const c32 a3 = cadd(u[3], u[7]);
   const c32 a4 = csub(u[0], u[4]);
   const c32 a5 = cmul_w1(csub(u[1], u[5]), sign);
   const c32 a6 = cmul_i (csub(u[2], u[6]), sign);
   const c32 a7 = cmul_w3(csub(u[3], u[7]), sign);

   const c32 b0 = cadd(a0, a2);
   const c32 b1 = cadd(a1, a3);
   const c32 b2 = csub(a0, a2);
   const c32 b3 = cmul_i(csub(a1, a3), sign);
   const c32 b4 = cadd(a4, a6);
   const c32 b5 = cadd(a5, a7);
   const c32 b6 = csub(a4, a6);
   const c32 b7 = cmul_i(csub(a5, a7), sign);

   v[0] = cadd(b0, b1);  v[4] = csub(b0, b1);
   v[2] = cadd(b2, b3);  v[6] = csub(b2, b3);
   v[1] = cadd(b4, b5);  v[5] = csub(b4, b5);
   v[3] = cadd(b6, b7);  v[7] = csub(b6, b7);
}

static void dft4(const c32* u, c32* v, int sign)
{
   const c32 a0 = cadd(u[0], u[2]);
   const c32 a1 = cadd(u[1], u[3]);
   const c32 a2 = csub(u[0], u[2]);
   const c32 a3 = cmul_i(csub(u[1], u[3]), sign);
   v[0] = cadd(a0, a1);  v[2] = csub(a0, a1);
   v[1] = cadd(a2, a3);  v[3] = csub(a2, a3);
}

static void dft2(const c32* u, c32* v)
{
   v[0] = cadd(u[0], u[1]);
   v[1] = csub(u[0], u[1]);
}

/* radix 16 = a radix-2 stage (x W16^k) feeding two radix-8s, outputs
 * interleaved even/odd (fufft.cuh:673-689) */
static void dft16(const c32* u, c32* v, int sign)
{
   c32 a[8], b[8], va[8], vb[8];
   for(int k = 0; k < 8; k++) {
      a[k] = cadd(u[k], u[k + 8]);
      b[k] = mul_w16(k, csub(u[k], u[k + 8]), sign);
   }
   dft8(a, va, sign);
   dft8(b, vb, sign);
   for(int k = 0; k < 8; k++) { v[2 * k] = va[k]; v[2 * k + 1] = vb[k]; }
}

static void dftR(int R, const c32* u, c32* v, int sign)
{
   switch(R) {
      case 2:  dft2(u, v); break;
      case 4:  dft4(u, v, sign); break;
      case 8:  dft8(u, v, sign); break;
      default: dft16(u, v, sign); break;
   }
}

/* ---- twiddles ------------------------------------------------------------ */

static void table_cs(int P, int64_t t, float* c, float* s)
{
   /* (float)cos/sin of 2*pi*t/P evaluated in double; the HIP library's host
    * code fills its device table with this same expression */
   const double th = 6.283185307179586476925286766559 * (double)t / (double)P;
   *c = (float)cos(th);
   *s = (float)sin(th);
}

void or_twiddle(int twmode, int sign, int P, int j, float* c, float* s)
{
   if(twmode == OR_TW_LIBM) {
      /* verify_kernel.cpp:31 with step from fufft.cuh:731 */
      const float step = (float)sign * 6.28318530717958647692f / (float)P;
      const float ang  = step * (float)j;
      *c = cosf(ang);
      *s = sinf(ang);
   } else {
      float sn;
      table_cs(P, j, c, &sn);
      *s = sign < 0 ? -sn : sn;
   }
}

/* fufft.cuh:436-450: w = W^j, then W^(jk) = W^(j(k-1)) * W^j */
static void tw_single(c32* x, int R, c32 w1)
{
   c32 w = w1;
   x[1] = cmul(x[1], w);
   for(int k = 2; k < R; k++) { w = cmul(w, w1); x[k] = cmul(x[k], w); }
}

/* fufft.cuh:701-720: v[2m] by (W^2)^m, v[2m+1] by W (W^2)^m */
static void tw_evenodd(c32* x, c32 w1)
{
   const c32 w2 = cmul(w1, w1);
   x[1] = cmul(x[1], w1);
   c32 ze = w2, zo = cmul(w2, w1);
   for(int m = 1; m < 8; m++) {
      x[2 * m]     = cmul(x[2 * m],     ze);
      x[2 * m + 1] = cmul(x[2 * m + 1], zo);
      if(m < 7) { ze = cmul(ze, w2); zo = cmul(zo, w2); }
   }
}

/* every stage twiddle read from the correctly rounded table: W_P^(jk), jk < P */
static void tw_direct(c32* x, int R, int P, int j, int sign)
{
   for(int k = 1; k < R; k++) {
      float c, s;
      table_cs(P, (int64_t)j * k, &c, &s);
      x[k] = cmul(x[k], mk(c, sign < 0 ? -s : s));
   }
}

static void apply_tw(c32* x, int R, int P, int j, int sign, int chain, int twmode)
{
   if(chain == OR_CHAIN_DIRECT) { tw_direct(x, R, P, j, sign); return; }
   c32 w1;
   or_twiddle(twmode, sign, P, j, &w1.x, &w1.y);
   if(chain == OR_CHAIN_EVENODD && R == 16) tw_evenodd(x, w1);
   else                                      tw_single(x, R, w1);
}

/* ---- passes -------------------------------------------------------------- */

/* One radix-R level, in place over groups (b, j): taps b*R*M + j + k*M.
 * DIF: butterfly then twiddle; DIT: twiddle then butterfly; no twiddle at
 * M == 1 (fufft.cuh:722-756, 1113-1140). */
void or_pass_f32(float* buf, int64_t len, int R, int M, int sign, int dit,
                 int chain, int twmode)
{
   c32* A = (c32*)buf;
   const int64_t ng = len / R;
   for(int64_t g = 0; g < ng; g++) {
      const int64_t j = g % M, b = g / M;
      const int64_t base = b * (int64_t)R * M + j;
      c32 u[16], v[16];
      for(int k = 0; k < R; k++) u[k] = A[base + (int64_t)k * M];
      if(dit && M > 1) apply_tw(u, R, R * M, (int)j, sign, chain, twmode);
      dftR(R, u, v, sign);
      if(!dit && M > 1) apply_tw(v, R, R * M, (int)j, sign, chain, twmode);
      for(int k = 0; k < R; k++) A[base + (int64_t)k * M] = v[k];
   }
}

/* column pass of an h x w image: the pass above along the row index, for
 * every column (verify_kernel.cpp:681-698) */
static void colpass(c32* A, int h, int w, int R, int m, int sign, int dit,
                    int chain, int twmode)
{
   for(int c = 0; c < w; c++)
      for(int g2 = 0; g2 < h / R; g2++) {
         const int j2 = g2 % m, b2 = g2 / m;
         const int64_t base = c + (int64_t)w * (b2 * R * m + j2);
         c32 u[16], v[16];
         for(int k = 0; k < R; k++) u[k] = A[base + (int64_t)k * w * m];
         if(dit && m > 1) apply_tw(u, R, R * m, j2, sign, chain, twmode);
         dftR(R, u, v, sign);
         if(!dit && m > 1) apply_tw(v, R, R * m, j2, sign, chain, twmode);
         for(int k = 0; k < R; k++) A[base + (int64_t)k * w * m] = v[k];
      }
}

static void dif_all(float* A, int n, const int* r, const int* ch, int np, int tw)
{
   int M = n;
   for(int i = 0; i < np; i++) { M /= r[i]; or_pass_f32(A, n, r[i], M, -1, 0, ch[i], tw); }
}

static void dit_all(float* A, int n, const int* r, const int* ch, int np, int tw)
{
   int M = 1;
   for(int i = np - 1; i >= 0; i--) { or_pass_f32(A, n, r[i], M, +1, 1, ch[i], tw); M *= r[i]; }
}

/* Mid policies (fufft.cuh:625-650) */
static void mid_apply(c32* A, const c32* f, int64_t n, int mid)
{
   if(mid == OR_MID_MUL) {
      for(int64_t i = 0; i < n; i++) A[i] = cmul(A[i], f[i]);
   } else if(mid == OR_MID_CONJ) {
      for(int64_t i = 0; i < n; i++) {
         const c32 x = A[i], y = f[i];
         A[i] = mk(fmaf(x.x, y.x, x.y * y.y), fmaf(x.y, y.x, -x.x * y.y));
      }
   }
}

/* ---- planning ------------------------------------------------------------ */

int or_factor(int n, int v, int* radices)
{
   int m = 0;
   while((1 << m) < n) m++;
   if((1 << m) != n || m < 1) return 0;
   int vb = 0;
   while((1 << vb) < v) vb++;
   const int a = m / vb, r = m % vb;
   int p = 0;
   if(r) radices[p++] = 1 << r;
   for(int i = 0; i < a; i++) radices[p++] = v;
   return p;
}

int or_mixedrev(int idx, const int* radices, int np)
{
   int w[OR_MAX_PASSES], m = 0;
   for(int i = 0; i < np; i++) {
      w[i] = 0;
      while((1 << w[i]) < radices[i]) w[i]++;
      m += w[i];
   }
   int d[OR_MAX_PASSES], pos = m;
   for(int i = 0; i < np; i++) { pos -= w[i]; d[i] = (idx >> pos) & ((1 << w[i]) - 1); }
   int out = 0, op = m;
   for(int i = np - 1; i >= 0; i--) { op -= w[i]; out |= d[i] << op; }
   return out;
}

/* ---- 1D conv, split fwd / apply, two-for-one ------------------------------ */

void or_conv_f32(const float* in, const float* filt, int64_t filt_stride,
                 float* out, int n, int64_t batch,
                 const int* radices, const int* chains, int np,
                 int mid, int twmode)
{
   for(int64_t t = 0; t < batch; t++) {
      float* A = out + 2 * t * n;
      if(A != in + 2 * t * n) memmove(A, in + 2 * t * n, sizeof(float) * 2 * (size_t)n);
      dif_all(A, n, radices, chains, np, twmode);
      mid_apply((c32*)A, (const c32*)(filt + 2 * t * filt_stride), n, mid);
      dit_all(A, n, radices, chains, np, twmode);
   }
}

void or_fwd_f32(const float* in, float* spec, int n, int64_t batch,
                const int* radices, const int* chains, int np, int twmode)
{
   for(int64_t t = 0; t < batch; t++) {
      float* A = spec + 2 * t * n;
      if(A != in + 2 * t * n) memmove(A, in + 2 * t * n, sizeof(float) * 2 * (size_t)n);
      dif_all(A, n, radices, chains, np, twmode);
   }
}

void or_apply_f32(const float* spec, int64_t spec_stride,
                  const float* filt, int64_t filt_stride, float* out,
                  int n, int64_t batch, const int* radices, const int* chains,
                  int np, int mid, int twmode)
{
   for(int64_t t = 0; t < batch; t++) {
      float* A = out + 2 * t * n;
      const float* S = spec + 2 * t * spec_stride;
      if(A != S) memmove(A, S, sizeof(float) * 2 * (size_t)n);
      mid_apply((c32*)A, (const c32*)(filt + 2 * t * filt_stride), n, mid);
      dit_all(A, n, radices, chains, np, twmode);
   }
}

void or_conv_r2_f32(const float* x, const float* y, const float* filt,
                    int64_t filt_stride, float* u, float* v, int n,
                    int64_t batch, const int* radices, const int* chains,
                    int np, int twmode)
{
   float* A = (float*)malloc(sizeof(float) * 2 * (size_t)n);
   for(int64_t t = 0; t < batch; t++) {
      for(int i = 0; i < n; i++) { A[2 * i] = x[t * n + i]; A[2 * i + 1] = y[t * n + i]; }
      dif_all(A, n, radices, chains, np, twmode);
      mid_apply((c32*)A, (const c32*)(filt + 2 * t * filt_stride), n, OR_MID_MUL);
      dit_all(A, n, radices, chains, np, twmode);
      for(int i = 0; i < n; i++) { u[t * n + i] = A[2 * i]; v[t * n + i] = A[2 * i + 1]; }
   }
   free(A);
}

/* ---- natural-order C2C ------------------------------------------------------
 * The reference's fufft_c2c (fufft.cuh:879-904; CPU transcription kernel_c2c,
 * verify_kernel.cpp:1183-1203) is a forward radix-8 Stockham transform.  This
 * build reaches natural order with the in-place passes instead: forward = the
 * DIF of the conv path, then slot s moved to bin mixedrev(s); inverse = bin
 * mixedrev(s) moved to slot s, then the DIT with sign +1, unnormalised.  The
 * permutation is exact, so the transform's rounding is that of the DIF / DIT
 * passes, which are pinned to the reference's transcription. */
void or_c2c_f32(const float* in, float* out, int n, int64_t batch,
                const int* radices, const int* chains, int np, int sign, int twmode)
{
   float* A = (float*)malloc(sizeof(float) * 2 * (size_t)n);
   int* rev = (int*)malloc(sizeof(int) * (size_t)n);
   for(int s = 0; s < n; s++) rev[s] = or_mixedrev(s, radices, np);
   for(int64_t t = 0; t < batch; t++) {
      const float* x = in + 2 * t * n;
      float* y = out + 2 * t * n;
      if(sign < 0) {
         memcpy(A, x, sizeof(float) * 2 * (size_t)n);
         dif_all(A, n, radices, chains, np, twmode);
         for(int s = 0; s < n; s++) { y[2 * rev[s]] = A[2 * s]; y[2 * rev[s] + 1] = A[2 * s + 1]; }
      } else {
         for(int s = 0; s < n; s++) { A[2 * s] = x[2 * rev[s]]; A[2 * s + 1] = x[2 * rev[s] + 1]; }
         dit_all(A, n, radices, chains, np, twmode);
         memcpy(y, A, sizeof(float) * 2 * (size_t)n);
      }
   }
   free(rev);
   free(A);
}

/* ---- 2D ------------------------------------------------------------------ */

static void rows_dif(float* A, int h, int w, const int* r, const int* ch, int np, int tw)
{
   int M = w;
   for(int i = 0; i < np; i++) { M /= r[i]; or_pass_f32(A, (int64_t)h * w, r[i], M, -1, 0, ch[i], tw); }
}

static void rows_dit(float* A, int h, int w, const int* r, const int* ch, int np, int tw)
{
   int M = 1;
   for(int i = np - 1; i >= 0; i--) { or_pass_f32(A, (int64_t)h * w, r[i], M, +1, 1, ch[i], tw); M *= r[i]; }
}

static void cols_dif(float* A, int h, int w, const int* r, const int* ch, int np, int tw)
{
   int m = h;
   for(int i = 0; i < np; i++) { m /= r[i]; colpass((c32*)A, h, w, r[i], m, -1, 0, ch[i], tw); }
}

static void cols_dit(float* A, int h, int w, const int* r, const int* ch, int np, int tw)
{
   int m = 1;
   for(int i = np - 1; i >= 0; i--) { colpass((c32*)A, h, w, r[i], m, +1, 1, ch[i], tw); m *= r[i]; }
}

void or_conv2d_f32(const float* in, const float* filt, int64_t filt_stride,
                   float* out, int h, int w, int64_t batch,
                   const int* rad_h, const int* ch_h, int nph,
                   const int* rad_w, const int* ch_w, int npw,
                   int mid, int twmode)
{
   const int64_t np = (int64_t)h * w;
   for(int64_t t = 0; t < batch; t++) {
      float* A = out + 2 * t * np;
      if(A != in + 2 * t * np) memmove(A, in + 2 * t * np, sizeof(float) * 2 * (size_t)np);
      rows_dif(A, h, w, rad_w, ch_w, npw, twmode);
      cols_dif(A, h, w, rad_h, ch_h, nph, twmode);
      mid_apply((c32*)A, (const c32*)(filt + 2 * t * filt_stride), np, mid);
      cols_dit(A, h, w, rad_h, ch_h, nph, twmode);
      rows_dit(A, h, w, rad_w, ch_w, npw, twmode);
   }
}

void or_fwd2d_f32(const float* in, float* spec, int h, int w, int64_t batch,
                  const int* rad_h, const int* ch_h, int nph,
                  const int* rad_w, const int* ch_w, int npw, int twmode)
{
   const int64_t np = (int64_t)h * w;
   for(int64_t t = 0; t < batch; t++) {
      float* A = spec + 2 * t * np;
      if(A != in + 2 * t * np) memmove(A, in + 2 * t * np, sizeof(float) * 2 * (size_t)np);
      rows_dif(A, h, w, rad_w, ch_w, npw, twmode);
      cols_dif(A, h, w, rad_h, ch_h, nph, twmode);
   }
}

void or_apply2d_f32(const float* spec, int64_t spec_stride, const float* filt,
                    int64_t filt_stride, float* out, int h, int w,
                    int64_t batch, const int* rad_h, const int* ch_h, int nph,
                    const int* rad_w, const int* ch_w, int npw, int mid,
                    int twmode)
{
   const int64_t np = (int64_t)h * w;
   for(int64_t t = 0; t < batch; t++) {
      float* A = out + 2 * t * np;
      const float* S = spec + 2 * t * spec_stride;
      if(A != S) memmove(A, S, sizeof(float) * 2 * (size_t)np);
      mid_apply((c32*)A, (const c32*)(filt + 2 * t * filt_stride), np, mid);
      cols_dit(A, h, w, rad_h, ch_h, nph, twmode);
      rows_dit(A, h, w, rad_w, ch_w, npw, twmode);
   }
}

/* ---- block floating point ------------------------------------------------ */

int or_bfp_exponent(float absmax)
{
   uint32_t bits;
   memcpy(&bits, &absmax, sizeof bits);
   bits &= 0x7fffffffu;
   const uint32_t xb = bits >> 23;
   if(xb == 0) return -128;                 /* zero or subnormal block */
   /* absmax = m * 2^(xb-126), m in [0.5, 1).  32767 * 2^(xb-141) >= absmax
    * iff m <= 32767/32768 iff the 23 fraction bits are <= 0x7ffe00. */
   int e = (int)xb - 141 + ((bits & 0x7fffffu) > 0x7ffe00u ? 1 : 0);
   return e < -128 ? -128 : e;
}

static float absmax_block(const float* x, int64_t npts)
{
   float m = 0.0f;
   for(int64_t i = 0; i < 2 * npts; i++) m = fmaxf(m, fabsf(x[i]));
   return m;
}

void or_bfp_quantize(const float* x, int64_t npts, int block,
                     int16_t* q, int8_t* e)
{
   for(int64_t b = 0; b < npts / block; b++) {
      const float* xb = x + 2 * b * block;
      const int ex = or_bfp_exponent(absmax_block(xb, block));
      e[b] = (int8_t)ex;
      for(int64_t i = 0; i < 2 * (int64_t)block; i++)
         q[2 * b * block + i] = (int16_t)rintf(ldexpf(xb[i], -ex));
   }
}

void or_bfp_dequantize(const int16_t* q, const int8_t* e, int64_t npts,
                       int block, float* x)
{
   for(int64_t b = 0; b < npts / block; b++)
      for(int64_t i = 0; i < 2 * (int64_t)block; i++)
         x[2 * b * block + i] = ldexpf((float)q[2 * b * block + i], e[b]);
}

void or_bfp_conv(const int16_t* qin, const int8_t* ein, const float* filt,
                 int64_t filt_stride, int16_t* qout, int8_t* eout, int n,
                 int64_t batch, int block, const int* radices,
                 const int* chains, int np, int mid, int twmode)
{
   float* A = (float*)malloc(sizeof(float) * 2 * (size_t)n);
   const int64_t nb = n / block;
   for(int64_t t = 0; t < batch; t++) {
      or_bfp_dequantize(qin + 2 * t * n, ein + t * nb, n, block, A);
      dif_all(A, n, radices, chains, np, twmode);
      mid_apply((c32*)A, (const c32*)(filt + 2 * t * filt_stride), n, mid);
      dit_all(A, n, radices, chains, np, twmode);
      or_bfp_quantize(A, n, block, qout + 2 * t * n, eout + t * nb);
   }
   free(A);
}

/* ---- fp64 ---------------------------------------------------------------- */

void or_fft2_f64(double* xd, int n, int sign)
{
   c64* x = (c64*)xd;
   for(int i = 1, j = 0; i < n; i++) {
      int bit = n >> 1;
      for(; j & bit; bit >>= 1) j ^= bit;
      j ^= bit;
      if(i < j) { const c64 t = x[i]; x[i] = x[j]; x[j] = t; }
   }
   /* twiddles straight from cos/sin per (len, k), via one table of W_n^t */
   double* ct = (double*)malloc(sizeof(double) * (size_t)(n / 2 + 1));
   double* st = (double*)malloc(sizeof(double) * (size_t)(n / 2 + 1));
   for(int t = 0; t < n / 2; t++) {
      const double th = 6.283185307179586476925286766559 * (double)t / (double)n;
      ct[t] = cos(th);
      st[t] = sign * sin(th);
   }
   for(int len = 2; len <= n; len <<= 1) {
      const int half = len / 2, step = n / len;
      for(int i = 0; i < n; i += len)
         for(int k = 0; k < half; k++) {
            const double wr = ct[k * step], wi = st[k * step];
            const c64 a0 = x[i + k], b = x[i + k + half];
            const c64 a1 = { b.x * wr - b.y * wi, b.x * wi + b.y * wr };
            x[i + k].x = a0.x + a1.x;        x[i + k].y = a0.y + a1.y;
            x[i + k + half].x = a0.x - a1.x; x[i + k + half].y = a0.y - a1.y;
         }
   }
   free(ct);
   free(st);
}

void or_conv_spec_f64(const float* a, const float* spec, int64_t spec_stride,
                      double* out, int n, int64_t batch, int mid)
{
   for(int64_t t = 0; t < batch; t++) {
      double* x = out + 2 * t * n;
      const float* s = spec + 2 * t * spec_stride;
      for(int i = 0; i < 2 * n; i++) x[i] = a[2 * t * n + i];
      or_fft2_f64(x, n, -1);
      for(int i = 0; i < n; i++) {
         const double xr = x[2 * i], xi = x[2 * i + 1];
         const double sr = s[2 * i], si = s[2 * i + 1];
         if(mid == OR_MID_MUL)       { x[2 * i] = xr * sr - xi * si; x[2 * i + 1] = xr * si + xi * sr; }
         else if(mid == OR_MID_CONJ) { x[2 * i] = xr * sr + xi * si; x[2 * i + 1] = xi * sr - xr * si; }
      }
      or_fft2_f64(x, n, +1);
   }
}

/* cpu_mixed.cpp fp64 butterflies, restated: generic complex arithmetic */
static inline c64 m64(double x, double y) { c64 r; r.x = x; r.y = y; return r; }
static inline c64 add64(c64 a, c64 b) { return m64(a.x + b.x, a.y + b.y); }
static inline c64 sub64(c64 a, c64 b) { return m64(a.x - b.x, a.y - b.y); }
static inline c64 mul64(c64 a, c64 b) { return m64(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x); }

static void dft8_64(const c64* u, c64* v, int sign)
{
   const double r2 = 0.70710678118654752440;
   const c64 w1 = m64(r2, sign * r2), w2 = m64(0.0, sign), w3 = m64(-r2, sign * r2);
   const c64 a0 = add64(u[0], u[4]), a1 = add64(u[1], u[5]);
   const c64 a2 = add64(u[2], u[6]), a3 = add64(u[3], u[7]);
   const c64 a4 = sub64(u[0], u[4]);
   const c64 a5 = mul64(sub64(u[1], u[5]), w1);
   const c64 a6 = mul64(sub64(u[2], u[6]), w2);
   const c64 a7 = mul64(sub64(u[3], u[7]), w3);
   const c64 b0 = add64(a0, a2), b1 = add64(a1, a3), b2 = sub64(a0, a2);
   const c64 b3 = mul64(sub64(a1, a3), w2);
   const c64 b4 = add64(a4, a6), b5 = add64(a5, a7), b6 = sub64(a4, a6);
   const c64 b7 = mul64(sub64(a5, a7), w2);
   v[0] = add64(b0, b1); v[4] = sub64(b0, b1);
   v[2] = add64(b2, b3); v[6] = sub64(b2, b3);
   v[1] = add64(b4, b5); v[5] = sub64(b4, b5);
   v[3] = add64(b6, b7); v[7] = sub64(b6, b7);
}

static void dftR_64(int R, const c64* u, c64* v, int sign)
{
   if(R == 2) { v[0] = add64(u[0], u[1]); v[1] = sub64(u[0], u[1]); return; }
   if(R == 4) {
      const c64 i2 = m64(0.0, sign);
      const c64 a0 = add64(u[0], u[2]), a1 = add64(u[1], u[3]);
      const c64 a2 = sub64(u[0], u[2]), a3 = mul64(sub64(u[1], u[3]), i2);
      v[0] = add64(a0, a1); v[2] = sub64(a0, a1); v[1] = add64(a2, a3); v[3] = sub64(a2, a3);
      return;
   }
   if(R == 8) { dft8_64(u, v, sign); return; }
   c64 a[8], b[8], va[8], vb[8];
   for(int i = 0; i < 8; i++) {
      const double ang = sign * 2.0 * 3.14159265358979323846 * (double)i / 16.0;
      a[i] = add64(u[i], u[i + 8]);
      b[i] = mul64(sub64(u[i], u[i + 8]), m64(cos(ang), sin(ang)));
   }
   dft8_64(a, va, sign);
   dft8_64(b, vb, sign);
   for(int k = 0; k < 8; k++) { v[2 * k] = va[k]; v[2 * k + 1] = vb[k]; }
}

/* cpu_mixed.cpp:116-153: every twiddle from its own cos/sin */
static void pass_64(c64* A, int n, int R, int M, int sign, int dit)
{
   for(int g = 0; g < n / R; g++) {
      const int b = g / M, j = g % M, base = b * R * M + j;
      c64 u[16], v[16];
      for(int k = 0; k < R; k++) u[k] = A[base + k * M];
      if(dit && M > 1)
         for(int k = 1; k < R; k++) {
            const double ang = sign * 2.0 * 3.14159265358979323846 * (double)(j * k) / (double)(R * M);
            u[k] = mul64(u[k], m64(cos(ang), sin(ang)));
         }
      dftR_64(R, u, v, sign);
      if(!dit && M > 1)
         for(int k = 1; k < R; k++) {
            const double ang = sign * 2.0 * 3.14159265358979323846 * (double)(j * k) / (double)(R * M);
            v[k] = mul64(v[k], m64(cos(ang), sin(ang)));
         }
      for(int k = 0; k < R; k++) A[base + k * M] = v[k];
   }
}

void or_mixed_conv_f64(const double* a, const double* spec_dr, double* out,
                       int n, int64_t batch, int v)
{
   int r[OR_MAX_PASSES];
   const int np = or_factor(n, v, r);
   for(int64_t t = 0; t < batch; t++) {
      c64* A = (c64*)(out + 2 * t * n);
      if((const double*)A != a + 2 * t * n) memmove(A, a + 2 * t * n, sizeof(double) * 2 * (size_t)n);
      int M = n;
      for(int i = 0; i < np; i++) { M /= r[i]; pass_64(A, n, r[i], M, -1, 0); }
      const c64* S = (const c64*)(spec_dr + 2 * t * n);
      for(int i = 0; i < n; i++) A[i] = mul64(A[i], S[i]);
      M = 1;
      for(int i = np - 1; i >= 0; i--) { pass_64(A, n, r[i], M, +1, 1); M *= r[i]; }
   }
}

double or_rel_l2_f32(const float* x, const float* y, int64_t ncomplex)
{
   double num = 0.0, den = 0.0;
   for(int64_t i = 0; i < 2 * ncomplex; i++) {
      const double d = (double)x[i] - (double)y[i];
      num += d * d;
      den += (double)y[i] * (double)y[i];
   }
   return den > 0.0 ? sqrt(num / den) : sqrt(num);
}

double or_rel_l2_f32_f64(const float* x, const double* y, int64_t ncomplex)
{
   double num = 0.0, den = 0.0;
   for(int64_t i = 0; i < 2 * ncomplex; i++) {
      const double d = (double)x[i] - y[i];
      num += d * d;
      den += y[i] * y[i];
   }
   return den > 0.0 ? sqrt(num / den) : sqrt(num);
}
