// Device-side building blocks of the fused cyclic-convolution kernels:
// complex arithmetic, radix-2/4/8/16 butterflies, stage twiddles, the LDS
// layout and the barrier used between passes.
//
// Arithmetic contract.  Every operation below is written in the same order,
// with the same explicit fmaf, as the reference's device code and its CPU
// transcription (fufft.cuh:208-450, 504-547, 652-720; verify_kernel.cpp:31-86,
// 1000-1011), and the library is compiled with -ffp-contract=off.  The only
// deliberate difference is the base twiddle W^j, which is read from a
// correctly-rounded fp32 table instead of __sincosf.  The CPU oracle
// (oracle/oracle.c, OR_TW_TABLE) follows the same contract, so kernel and
// oracle agree bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fufft {

// ---- constants (fufft.cuh:40, 517-518) --------------------------------------
#define FUFFT_R2  0.70710678118654752440f
#define FUFFT_C16 0.92387953251128673848f
#define FUFFT_S16 0.38268343236508977173f

// ---- complex primitives -----------------------------------------------------
__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }

// 2 MUL + 2 FMA (fufft.cuh:255-260)
__device__ __forceinline__ float2 cmul(float2 a, float2 b)
{
   return make_float2(__builtin_fmaf(a.x, b.x, -a.y * b.y),
                      __builtin_fmaf(a.x, b.y,  a.y * b.x));
}

// a * conj(b): the correlation mid operation (fufft.cuh:641-649)
__device__ __forceinline__ float2 cmul_conj(float2 x, float2 y)
{
   return make_float2(__builtin_fmaf(x.x, y.x,  x.y * y.y),
                      __builtin_fmaf(x.y, y.x, -x.x * y.y));
}

// x (+-i): a swap and a sign flip, no arithmetic
template<int SIGN>
__device__ __forceinline__ float2 cmul_i(float2 a)
{
   return SIGN < 0 ? make_float2(a.y, -a.x) : make_float2(-a.y, a.x);
}

// x W8^1 = r2 (1, SIGN): 2 add + 2 mul
template<int SIGN>
__device__ __forceinline__ float2 cmul_w1(float2 a)
{
   return SIGN < 0 ? make_float2(FUFFT_R2 * (a.x + a.y), FUFFT_R2 * (a.y - a.x))
                   : make_float2(FUFFT_R2 * (a.x - a.y), FUFFT_R2 * (a.x + a.y));
}

// x W8^3 = r2 (-1, SIGN)
template<int SIGN>
__device__ __forceinline__ float2 cmul_w3(float2 a)
{
   return SIGN < 0 ? make_float2(FUFFT_R2 * (a.y - a.x), FUFFT_R2 * (-a.x - a.y))
                   : make_float2(FUFFT_R2 * (-a.x - a.y), FUFFT_R2 * (a.x - a.y));
}

// x W16^K
template<int K, int SIGN>
__device__ __forceinline__ float2 mul_w16(float2 x)
{
   constexpr float s = (float)SIGN;
   if constexpr(K == 0) return x;
   else if constexpr(K == 1) return cmul(x, make_float2( FUFFT_C16, s * FUFFT_S16));
   else if constexpr(K == 2) return cmul_w1<SIGN>(x);
   else if constexpr(K == 3) return cmul(x, make_float2( FUFFT_S16, s * FUFFT_C16));
   else if constexpr(K == 4) return cmul_i<SIGN>(x);
   else if constexpr(K == 5) return cmul(x, make_float2(-FUFFT_S16, s * FUFFT_C16));
   else if constexpr(K == 6) return cmul_w3<SIGN>(x);
   else                      return cmul(x, make_float2(-FUFFT_C16, s * FUFFT_S16));
}

// ---- butterflies on a register array ---------------------------------------
// Each takes the R taps of one group, u[k] = r[OFF + k*STRIDE], and writes the
// natural-order outputs back to the same registers.  All indices are
// compile-time constants, so the arrays live in VGPRs.

template<int SIGN, int OFF, int STRIDE, int NR>
__device__ __forceinline__ void dft2(float2 (&r)[NR])
{
   const float2 u0 = r[OFF], u1 = r[OFF + STRIDE];
   r[OFF]          = cadd(u0, u1);
   r[OFF + STRIDE] = csub(u0, u1);
}

template<int SIGN, int OFF, int STRIDE, int NR>
__device__ __forceinline__ void dft4(float2 (&r)[NR])
{
   const float2 u0 = r[OFF], u1 = r[OFF + STRIDE], u2 = r[OFF + 2 * STRIDE], u3 = r[OFF + 3 * STRIDE];
   const float2 a0 = cadd(u0, u2), a1 = cadd(u1, u3);
   const float2 a2 = csub(u0, u2), a3 = cmul_i<SIGN>(csub(u1, u3));
   r[OFF]              = cadd(a0, a1);
   r[OFF + 2 * STRIDE] = csub(a0, a1);
   r[OFF + STRIDE]     = cadd(a2, a3);
   r[OFF + 3 * STRIDE] = csub(a2, a3);
}

// radix 8 as three radix-2 stages (fufft.cuh:377-405)
template<int SIGN>
__device__ __forceinline__ void dft8v(const float2* u, float2* v)
{
   const float2 a0 = cadd(u[0], u[4]);
   const float2 a1 = cadd(u[1], u[5]);
   const float2 a2 = cadd(u[2], u[6]);
   const float2 a3 = cadd(u[3], u[7]);
   const float2 a4 = csub(u[0], u[4]);
   const float2 a5 = cmul_w1<SIGN>(csub(u[1], u[5]));
   const float2 a6 = cmul_i <SIGN>(csub(u[2], u[6]));
   const float2 a7 = cmul_w3<SIGN>(csub(u[3], u[7]));

   const float2 b0 = cadd(a0, a2);
   const float2 b1 = cadd(a1, a3);
   const float2 b2 = csub(a0, a2);
   const float2 b3 = cmul_i<SIGN>(csub(a1, a3));
   const float2 b4 = cadd(a4, a6);
   const float2 b5 = cadd(a5, a7);
   const float2 b6 = csub(a4, a6);
   const float2 b7 = cmul_i<SIGN>(csub(a5, a7));

   v[0] = cadd(b0, b1);  v[4] = csub(b0, b1);
   v[2] = cadd(b2, b3);  v[6] = csub(b2, b3);
   v[1] = cadd(b4, b5);  v[5] = csub(b4, b5);
   v[3] = cadd(b6, b7);  v[7] = csub(b6, b7);
}

template<int SIGN, int OFF, int STRIDE, int NR>
__device__ __forceinline__ void dft8(float2 (&r)[NR])
{
   float2 u[8], v[8];
#pragma unroll
   for(int k = 0; k < 8; k++) u[k] = r[OFF + k * STRIDE];
   dft8v<SIGN>(u, v);
#pragma unroll
   for(int k = 0; k < 8; k++) r[OFF + k * STRIDE] = v[k];
}

// radix 16 = one radix-2 stage (x W16^k) feeding two radix-8s; outputs
// interleave even/odd (fufft.cuh:673-689)
template<int SIGN, int OFF, int STRIDE, int NR>
__device__ __forceinline__ void dft16(float2 (&r)[NR])
{
   float2 a[8], b[8], va[8], vb[8];
#define FUFFT_R2STEP(K)                                                             \
   a[K] = cadd(r[OFF + (K) * STRIDE], r[OFF + ((K) + 8) * STRIDE]);                \
   b[K] = mul_w16<K, SIGN>(csub(r[OFF + (K) * STRIDE], r[OFF + ((K) + 8) * STRIDE]));
   FUFFT_R2STEP(0) FUFFT_R2STEP(1) FUFFT_R2STEP(2) FUFFT_R2STEP(3)
   FUFFT_R2STEP(4) FUFFT_R2STEP(5) FUFFT_R2STEP(6) FUFFT_R2STEP(7)
#undef FUFFT_R2STEP
   dft8v<SIGN>(a, va);
   dft8v<SIGN>(b, vb);
#pragma unroll
   for(int k = 0; k < 8; k++) { r[OFF + (2 * k) * STRIDE] = va[k]; r[OFF + (2 * k + 1) * STRIDE] = vb[k]; }
}

template<int R, int SIGN, int OFF, int STRIDE, int NR>
__device__ __forceinline__ void dftR(float2 (&r)[NR])
{
   if constexpr(R == 2)       dft2 <SIGN, OFF, STRIDE>(r);
   else if constexpr(R == 4)  dft4 <SIGN, OFF, STRIDE>(r);
   else if constexpr(R == 8)  dft8 <SIGN, OFF, STRIDE>(r);
   else                       dft16<SIGN, OFF, STRIDE>(r);
}

// ---- twiddles ----------------------------------------------------------------
// The table holds, for every power of two P in [2, 2^FUFFT_TW_LOG_MAX], the P
// entries (cos, sin)(2*pi*t/P) at offset P; entry 0..1 are unused.  A stage
// twiddle of a radix-R pass at stride M is W_{R*M}^j, so W^j = tw[R*M + j].
#define FUFFT_TW_LOG_MAX 20
#define FUFFT_TW_ENTRIES (2u << FUFFT_TW_LOG_MAX)


template<int SIGN>
__device__ __forceinline__ float2 tw_load(const float2* __restrict__ tw, int idx)
{
   const float2 w = tw[idx];
   return SIGN < 0 ? make_float2(w.x, -w.y) : w;
}

// single chain, W^(jk) = W^(j(k-1)) * W^j  (fufft.cuh:436-450)
template<int R, int OFF, int STRIDE, int NR>
__device__ __forceinline__ void tw_single(float2 (&r)[NR], float2 w1)
{
   float2 w = w1;
   r[OFF + STRIDE] = cmul(r[OFF + STRIDE], w);
#pragma unroll
   for(int k = 2; k < R; k++) { w = cmul(w, w1); r[OFF + k * STRIDE] = cmul(r[OFF + k * STRIDE], w); }
}

// the single chain that also hands back the powers it generated, w[k] = W^(jk)
template<int R, int OFF, int STRIDE, int NR>
__device__ __forceinline__ void tw_single_keep(float2 (&r)[NR], float2 w1, float2 (&w)[R])
{
   w[1] = w1;
   r[OFF + STRIDE] = cmul(r[OFF + STRIDE], w1);
#pragma unroll
   for(int k = 2; k < R; k++) { w[k] = cmul(w[k - 1], w1); r[OFF + k * STRIDE] = cmul(r[OFF + k * STRIDE], w[k]); }
}

// Multiply by the conjugates of powers a forward chain generated.  The forward
// chain runs on conj(W^j), the inverse's on W^j, and a product of conjugates
// is the conjugate of the product bit for bit (each fma only changes sign), so
// conj(w[k]) equals the inverse chain's W^(jk) exactly.
template<int R, int OFF, int STRIDE, int NR>
__device__ __forceinline__ void tw_kept_conj(float2 (&r)[NR], const float2 (&w)[R])
{
#pragma unroll
   for(int k = 1; k < R; k++) r[OFF + k * STRIDE] = cmul(r[OFF + k * STRIDE], make_float2(w[k].x, -w[k].y));
}

// radix 16: even outputs by (W^2)^m, odd by W (W^2)^m -- two 7-step chains
// (fufft.cuh:701-720)
template<int OFF, int STRIDE, int NR>
__device__ __forceinline__ void tw_evenodd(float2 (&r)[NR], float2 w1)
{
   const float2 w2 = cmul(w1, w1);
   r[OFF + STRIDE] = cmul(r[OFF + STRIDE], w1);
   float2 ze = w2, zo = cmul(w2, w1);
#pragma unroll
   for(int m = 1; m < 8; m++) {
      r[OFF + 2 * m * STRIDE]       = cmul(r[OFF + 2 * m * STRIDE], ze);
      r[OFF + (2 * m + 1) * STRIDE] = cmul(r[OFF + (2 * m + 1) * STRIDE], zo);
      if(m < 7) { ze = cmul(ze, w2); zo = cmul(zo, w2); }
   }
}

// the even/odd chains that also hand back the powers they generated, w[k] = W^(jk)
template<int OFF, int STRIDE, int NR>
__device__ __forceinline__ void tw_evenodd_keep(float2 (&r)[NR], float2 w1, float2 (&w)[16])
{
   const float2 w2 = cmul(w1, w1);
   w[1] = w1;
   w[2] = w2;
   r[OFF + STRIDE] = cmul(r[OFF + STRIDE], w1);
   float2 ze = w2, zo = cmul(w2, w1);
   w[3] = zo;
#pragma unroll
   for(int m = 1; m < 8; m++) {
      r[OFF + 2 * m * STRIDE]       = cmul(r[OFF + 2 * m * STRIDE], ze);
      r[OFF + (2 * m + 1) * STRIDE] = cmul(r[OFF + (2 * m + 1) * STRIDE], zo);
      if(m < 7) { ze = cmul(ze, w2); zo = cmul(zo, w2); w[2 * m + 2] = ze; w[2 * m + 3] = zo; }
   }
}

// chain selection: in-workgroup radix-16 passes use the even/odd chains, every
// other pass (lead radices, the four-step outer radix-16 level) the single
// chain -- exactly as in the reference's kernels
enum { CHAIN_SINGLE = 0, CHAIN_EVENODD = 1 };

template<int R, int CHAIN, int OFF, int STRIDE, int NR>
__device__ __forceinline__ void twiddle_group(float2 (&r)[NR], float2 w1)
{
   if constexpr(R == 16 && CHAIN == CHAIN_EVENODD) tw_evenodd<OFF, STRIDE>(r, w1);
   else                                             tw_single<R, OFF, STRIDE>(r, w1);
}

// ---- buffer-resource memory access ---------------------------------------------------
// Global traffic goes through raw buffer instructions: the base address lives in
// a wave-uniform 128-bit resource (SGPRs), each lane supplies one 32-bit byte
// offset, and per-tap offsets ride in the scalar offset field, so a lane keeps
// one VGPR of addressing instead of a 64-bit pointer per tap.  Accesses beyond
// num_records bytes read zero and drop writes.
// cache policy of a buffer access on gfx950: NT (bit 1) streams data that is
// touched once -- a signal read and a result written -- past the caches, so
// they stay with data that is reused (the filter, twiddles, LDS spills).
// Measured on the 1D conv and BFP kernels at every size: +2 to +3.5%, and on
// a plain copy 5.5 -> 6.2 TB/s.  The four-step middle does not use it: its
// data is read again by the next launch from the last-level cache.
enum { POL_DEFAULT = 0, POL_NT = 2 };

struct Buf {
   __amdgpu_buffer_rsrc_t r;
   // dword 3 of the resource: 32-bit data format, as gfx9 untyped access expects
   static constexpr int kFlags = 0x00020000;

   __device__ __forceinline__ Buf(const void* base, uint32_t bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kFlags)) {}

   __device__ __forceinline__ float ld1(uint32_t voff, uint32_t soff) const
   {
      return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
   }
   template<int POL = POL_DEFAULT>
   __device__ __forceinline__ float2 ld2(uint32_t voff, uint32_t soff) const
   {
      return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, POL));
   }
   template<int POL = POL_DEFAULT>
   __device__ __forceinline__ float4 ld4(uint32_t voff, uint32_t soff) const
   {
      return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, POL));
   }
   template<int POL = POL_DEFAULT>
   __device__ __forceinline__ uint32_t ldu(uint32_t voff, uint32_t soff) const
   {
      return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, POL);
   }
   __device__ __forceinline__ int ldi8(uint32_t voff, uint32_t soff) const
   {
      return (int)(int8_t)__builtin_amdgcn_raw_buffer_load_b8(r, voff, soff, 0);
   }
   __device__ __forceinline__ void st1(float v, uint32_t voff, uint32_t soff) const
   {
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, voff, soff, 0);
   }
   template<int POL = POL_DEFAULT>
   __device__ __forceinline__ void st2(float2 v, uint32_t voff, uint32_t soff) const
   {
      typedef uint32_t u2 __attribute__((ext_vector_type(2)));
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, v), r, voff, soff, POL);
   }
   __device__ __forceinline__ void st4(float4 v, uint32_t voff, uint32_t soff) const
   {
      typedef uint32_t u4 __attribute__((ext_vector_type(4)));
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), r, voff, soff, 0);
   }
   template<int POL = POL_DEFAULT>
   __device__ __forceinline__ void stu(uint32_t v, uint32_t voff, uint32_t soff) const
   {
      __builtin_amdgcn_raw_buffer_store_b32(v, r, voff, soff, POL);
   }
};

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// t % count for the filter and spectrum counts the entry points produce: one
// shared array (1), one per transform (count >= the launch's transforms, so
// t < count), or one per chunk of a four-step transform (a power of two).
// Three VALU operations instead of a runtime integer division (about a dozen);
// the launchers reject any other count (modulo_count_ok).
__device__ __forceinline__ uint32_t modulo_count(uint32_t t, uint32_t count)
{
   return t < count ? t : t & (count - 1u);
}

__host__ __device__ constexpr bool modulo_count_ok(uint32_t count, uint32_t ntrans)
{
   return count != 0 && (count >= ntrans || (count & (count - 1u)) == 0);
}

// ---- synchronisation between passes -------------------------------------------
// A transform held by one wavefront needs no s_barrier: LDS operations of a
// wave execute in order, so a wavefront-scope fence (which stops the compiler
// from moving LDS accesses across it) is enough.  Wider transforms use the
// workgroup barrier; such workgroups hold exactly one transform.
template<int LANES>
__device__ __forceinline__ void pass_barrier()
{
   if constexpr(LANES <= 64) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
   } else {
      __syncthreads();
   }
}

}  // namespace fufft
