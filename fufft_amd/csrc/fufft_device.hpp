// Device-side building blocks of the fused cyclic-convolution kernels:
// complex arithmetic, radix-2/4/8/16 butterflies, stage twiddles, the LDS
// layout and the barrier used between passes.
//
// Arithmetic contract.  Every rounded operation below (an add, a product, an
// explicit fmaf) takes the operands the matching step of the reference's
// device code and CPU transcription takes (fufft.cuh:208-450, 504-547,
// 652-720; verify_kernel.cpp:31-86, 1000-1011): the same radix-2 stages, the
// same constant rotations and the same twiddle recurrences, here written as
// generic networks over compile-time indices.  The library is compiled with
// -ffp-contract=off.  The only deliberate difference is the base twiddle W^j,
// which is read from a correctly-rounded fp32 table instead of __sincosf.  The
// CPU oracle (oracle/oracle.c, OR_TW_TABLE) follows the same contract, so
// kernel and oracle agree bit for bit.
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

// x * W16^E, W16 = exp(SIGN 2 pi i / 16), E = 0..7: every stage twiddle of
// a radix-2 network of at most 16 points is one of these.  A quarter turn
// (E = 4) is a swap and a sign; the odd eighths (E = 2, 6) are
// sqrt(1/2) (+-1 + SIGN i), one add per component and a scale; the odd
// sixteenths are a general product with (cos, SIGN sin)(2 pi E / 16).
// Each rounding step has the operands of the reference's MULTIPLY forms
// (fufft.cuh:266-340, 534-547).
template<int E, int SIGN>
__device__ __forceinline__ float2 rot16(float2 x)
{
   static_assert(E >= 0 && E < 8, "rot16: E in 0..7");
   constexpr float s = (float)SIGN;
   if constexpr(E == 0) {
      return x;
   } else if constexpr(E == 4) {
      return make_float2(-s * x.y, s * x.x);
   } else if constexpr(E == 2) {
      // sqrt(1/2) (1 + SIGN i): one add or subtract per component, then the scale
      return SIGN < 0 ? make_float2(FUFFT_R2 * (x.x + x.y), FUFFT_R2 * (x.y - x.x))
                      : make_float2(FUFFT_R2 * (x.x - x.y), FUFFT_R2 * (x.x + x.y));
   } else if constexpr(E == 6) {
      // sqrt(1/2) (-1 + SIGN i)
      return SIGN < 0 ? make_float2(FUFFT_R2 * (x.y - x.x), FUFFT_R2 * (-x.x - x.y))
                      : make_float2(FUFFT_R2 * (-x.x - x.y), FUFFT_R2 * (x.x - x.y));
   } else {
      constexpr float cs = E == 1 ? FUFFT_C16 : E == 3 ? FUFFT_S16 : E == 5 ? -FUFFT_S16 : -FUFFT_C16;
      constexpr float sn = E == 1 ? FUFFT_S16 : E == 3 ? FUFFT_C16 : E == 5 ?  FUFFT_C16 :  FUFFT_S16;
      return cmul(x, make_float2(cs, s * sn));
   }
}

// ---- butterflies on a register array ---------------------------------------
// An R-point DFT (R = 2, 4, 8, 16) of the taps u[k] = r[OFF + k*STRIDE], in
// place, as log2(R) radix-2 decimation-in-frequency stages.  The stage of
// half-width H maps each pair (x[k], x[k+H]) of a block of 2H to
// (x[k] + x[k+H], (x[k] - x[k+H]) W_{2H}^k), and W_{2H}^k = W16^(8k/H).
// After the last stage position p holds frequency bitrev(p), so the values
// go back to the taps through that reversal and leave in natural order.
// All indices are compile-time constants: the values stay in VGPRs.
//
// The order the butterflies are written in is the order the compiler's
// scheduler starts from, and it shows in registers and time (up to 1.5%,
// same box, bit-identical results).  The order kept: a network of 16 points
// runs its first stage pair by pair and then each half to the end before the
// other starts; a network of up to 8 points goes stage by stage, each block's
// sums before its differences.

// one block of 2H values from B: the H sums, then the H rotated differences
template<int SIGN, int R, int B, int H, int K = 0>
__device__ __forceinline__ void r2_sums(const float2 (&x)[R], float2 (&s)[H])
{
   if constexpr(K < H) {
      s[K] = cadd(x[B + K], x[B + K + H]);
      r2_sums<SIGN, R, B, H, K + 1>(x, s);
   }
}

template<int SIGN, int R, int B, int H, int K = 0>
__device__ __forceinline__ void r2_diffs(float2 (&x)[R])
{
   if constexpr(K < H) {
      x[B + K + H] = rot16<K * 8 / H, SIGN>(csub(x[B + K], x[B + K + H]));
      r2_diffs<SIGN, R, B, H, K + 1>(x);
   }
}

// one block, pair by pair: the sum and the rotated difference of pair K
template<int SIGN, int R, int B, int H, int K = 0>
__device__ __forceinline__ void r2_paired(float2 (&x)[R])
{
   if constexpr(K < H) {
      const float2 sum = cadd(x[B + K], x[B + K + H]);
      x[B + K + H] = rot16<K * 8 / H, SIGN>(csub(x[B + K], x[B + K + H]));
      x[B + K] = sum;
      r2_paired<SIGN, R, B, H, K + 1>(x);
   }
}

// one stage of half-width H over the blocks B0, B0 + 2H, ... below B0 + SPAN
template<int SIGN, int R, int H, int B0, int SPAN, int B = B0>
__device__ __forceinline__ void r2_stage(float2 (&x)[R])
{
   if constexpr(B < B0 + SPAN) {
      if constexpr(SPAN > 8) {
         r2_paired<SIGN, R, B, H>(x);
      } else {
         float2 s[H];
         r2_sums<SIGN, R, B, H>(x, s);
         r2_diffs<SIGN, R, B, H>(x);
#pragma unroll
         for(int k = 0; k < H; k++) x[B + k] = s[k];
      }
      r2_stage<SIGN, R, H, B0, SPAN, B + 2 * H>(x);
   }
}

// the network on the SPAN values from B0
template<int SIGN, int R, int B0 = 0, int SPAN = R, int H = SPAN / 2>
__device__ __forceinline__ void r2_network(float2 (&x)[R])
{
   if constexpr(H >= 1) {
      r2_stage<SIGN, R, H, B0, SPAN>(x);
      if constexpr(SPAN > 8) {
         r2_network<SIGN, R, B0, SPAN / 2>(x);
         r2_network<SIGN, R, B0 + SPAN / 2, SPAN / 2>(x);
      } else {
         r2_network<SIGN, R, B0, SPAN, H / 2>(x);
      }
   }
}

constexpr int bitrev_of(int p, int bits) { return bits == 0 ? 0 : ((p & 1) << (bits - 1)) | bitrev_of(p >> 1, bits - 1); }
constexpr int log2_of(int r) { return r <= 1 ? 0 : 1 + log2_of(r >> 1); }

template<int R, int SIGN, int OFF, int STRIDE, int NR>
__device__ __forceinline__ void dftR(float2 (&r)[NR])
{
   static_assert(R == 2 || R == 4 || R == 8 || R == 16, "dftR: radix 2, 4, 8 or 16");
   float2 x[R];
#pragma unroll
   for(int k = 0; k < R; k++) x[k] = r[OFF + k * STRIDE];
   r2_network<SIGN, R>(x);
#pragma unroll
   for(int p = 0; p < R; p++) r[OFF + bitrev_of(p, log2_of(R)) * STRIDE] = x[p];
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

// A pass multiplies tap k of a group by W^(jk), from a recurrence on the
// table's W^j, so each product has the reference's operands.  With KEEP the
// chains hand back the powers they made, pw[k] = W^(jk), for a pass that
// needs the same twiddles conjugated (tw_kept_conj); the single chain keeps
// its state there in any case, a local array the compiler drops.
//  - one chain, pw[k] = pw[k-1] W^j (fufft.cuh:436-450), at every radix;
//  - inside a workgroup at radix 16, one chain per tap parity: tap 2m + q
//    takes W^(2j) times tap 2m - 2 + q's power, from W^(2j) and W^(3j), 7
//    steps deep instead of 14 (fufft.cuh:701-720).
// The forms below (the single chain's state in pw, the parity chains'
// running pair) are the ones the kernels were measured with: other forms of
// the same recurrences schedule differently, up to 1.5% slower.
template<int R, int OFF, int STRIDE, int NR>
__device__ __forceinline__ void chain_one(float2 (&r)[NR], float2 w1, float2 (&pw)[R])
{
   pw[1] = w1;
   r[OFF + STRIDE] = cmul(r[OFF + STRIDE], w1);
#pragma unroll
   for(int k = 2; k < R; k++) {
      pw[k] = cmul(pw[k - 1], w1);
      r[OFF + k * STRIDE] = cmul(r[OFF + k * STRIDE], pw[k]);
   }
}

template<int OFF, int STRIDE, bool KEEP, int NR>
__device__ __forceinline__ void chain_parity(float2 (&r)[NR], float2 w1, float2 (&pw)[16])
{
   const float2 sq = cmul(w1, w1);
   if constexpr(KEEP) { pw[1] = w1; pw[2] = sq; }
   r[OFF + STRIDE] = cmul(r[OFF + STRIDE], w1);
   float2 run[2] = {sq, cmul(sq, w1)};   // the powers of the even and odd taps
   if constexpr(KEEP) pw[3] = run[1];
#pragma unroll
   for(int m = 1; m < 8; m++) {
#pragma unroll
      for(int q = 0; q < 2; q++) r[OFF + (2 * m + q) * STRIDE] = cmul(r[OFF + (2 * m + q) * STRIDE], run[q]);
      if(m < 7) {
#pragma unroll
         for(int q = 0; q < 2; q++) run[q] = cmul(run[q], sq);
         if constexpr(KEEP) {
#pragma unroll
            for(int q = 0; q < 2; q++) pw[2 * m + 2 + q] = run[q];
         }
      }
   }
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

// chain selection: in-workgroup radix-16 passes use the parity chains, every
// other pass (lead radices, the four-step outer radix-16 level) the single
// chain, as the reference's kernels do
enum { CHAIN_SINGLE = 0, CHAIN_EVENODD = 1 };

template<int R, int CHAIN, int OFF, int STRIDE, int NR>
__device__ __forceinline__ void twiddle_group(float2 (&r)[NR], float2 w1)
{
   float2 pw[R];
   if constexpr(R == 16 && CHAIN == CHAIN_EVENODD) chain_parity<OFF, STRIDE, false>(r, w1, pw);
   else                                             chain_one<R, OFF, STRIDE>(r, w1, pw);
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
