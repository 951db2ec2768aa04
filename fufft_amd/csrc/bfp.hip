// int16 block-floating-point fused convolution for gfx950.
//
// Replaces fufft_pipeline_v16_bfp (fufft.cuh:1614-1701).  HBM carries 4 bytes
// per point (int16 re in the low halfword, int16 im in the high halfword) plus
// one int8 exponent per block of 64 consecutive points; all arithmetic in
// between is the fp32 pipeline of conv1d.hip, bit for bit.  The reference
// keeps one fp32 scale per transform and an int16 filter; here the filter is
// fp32 and the exponent rule is
//    e = -128 for an all-zero (or subnormal) block, else the smallest integer
//        with absmax <= 32767 * 2^e, clamped at -128;   q = rint(x * 2^-e).
// A block is B consecutive points of a signal, B a power of two from 64 to N
// (B = N: one exponent per signal, the reference's per-transform scale).
//
// Mapping: a transform has T = N/V >= 64 lanes, and register q of a wavefront
// holds the 64 consecutive points 64*w + q*T .. (w = wavefront index within
// the transform), all inside one block.  So input exponents are uniform per
// (wavefront, register), and the V abs-maxima of a wavefront's registers come
// from one transposed cross-lane reduction.  With B = 64 each of them is a
// block's maximum: no LDS pass and no workgroup barrier for the scale, unlike
// the reference's shared-memory atomicMax rendezvous (fufft.cuh:1674-1692).
// With B > 64 a block spans several (wavefront, register) pairs, and their
// maxima meet in one LDS atomic max per pair (the reference's rendezvous,
// on V values per wavefront instead of every element).
#include "fufft_device.hpp"
#include "fufft_plan.hpp"
#include "fufft_internal.hpp"

namespace fufft {

constexpr int bfp_cpb(int T) { return T >= 128 ? 1 : 256 / T; }

// exponent of a block from its abs-max bits (see the rule above); every
// operation is exact, so it agrees with the host codec and the CPU oracle
__device__ __forceinline__ int bfp_exponent_bits(uint32_t bits)
{
   bits &= 0x7fffffffu;
   const int xb = (int)(bits >> 23);
   int e = xb - 141 + ((bits & 0x7fffffu) > 0x7ffe00u ? 1 : 0);
   e = e < -128 ? -128 : e;
   return xb == 0 ? -128 : e;
}

// ---- block maxima across a wavefront ------------------------------------------------
// The V registers of a wavefront are V blocks; their maxima are found with one
// transposed reduction instead of V full-wave reductions.  Values are the bits
// of non-negative floats, so unsigned compares order them exactly and the DPP
// lane moves fold into v_max_u32_dpp.

template<int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v)
{
   return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, true);
}

__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

// partner lane for level S: xor 1, xor 2 (quad_perm), then rotations by 4 and
// 8 within a row of 16.  A rotation by 4 is not an involution, but the partner
// always has the opposite bit 2 and the same bits 0-1, and the rotation by 8
// that follows joins the remaining quads, so every lane still sees all 16.
template<int S>
__device__ __forceinline__ uint32_t level_partner(uint32_t v)
{
   if constexpr(S == 0)      return dpp_u<0xB1>(v);    // quad_perm [1,0,3,2]
   else if constexpr(S == 1) return dpp_u<0x4E>(v);    // quad_perm [2,3,0,1]
   else if constexpr(S == 2) return dpp_u<0x124>(v);   // row_ror:4
   else                      return dpp_u<0x128>(v);   // row_ror:8 (= xor 8)
}

__device__ __forceinline__ uint32_t swap_max16(uint32_t v)
{
   const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);   // rows 0<->1, 2<->3
   return umax(r[0], r[1]);
}

__device__ __forceinline__ uint32_t swap_max32(uint32_t v)
{
   const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);   // halves swapped
   return umax(r[0], r[1]);
}

// On return lane l holds the wavefront maximum of m[l % V].  Level s halves
// the register count: lanes with bit s clear keep the even register of each
// pair and receive their partner's even register; lanes with bit s set keep
// and receive the odd one.  The lane bits left over after log2(V) levels
// reduce plainly.
template<int V>
__device__ __forceinline__ uint32_t block_maxima(uint32_t (&m)[V], uint32_t lane)
{
   constexpr int LOGV = V == 16 ? 4 : 3;
   static_assert(V == 8 || V == 16, "one register per block level");
   static_for<LOGV>([&](auto si) {
      constexpr int S = decltype(si)::value;
      constexpr int K = V >> S;
      const bool hi = (lane >> S) & 1u;
#pragma unroll
      for(int i = 0; i < K / 2; i++) {
         const uint32_t keep = hi ? m[2 * i + 1] : m[2 * i];
         const uint32_t send = hi ? m[2 * i] : m[2 * i + 1];
         m[i] = umax(keep, level_partner<S>(send));
      }
   });
   uint32_t x = m[0];
   if constexpr(LOGV == 3) x = umax(x, dpp_u<0x128>(x));
   return swap_max32(swap_max16(x));
}

// bmax words per transform for blocks of 128 points or more
constexpr int bfp_bmax_words(int n) { return n / 128; }

// Radix-8 lanes run 8 wavefronts per SIMD within 64 VGPRs.  Without the hint
// the long-block epilogue (N = 4096) and the radix-8 N = 8192 plan allocate
// 71, i.e. 7 wavefronts per SIMD (for N = 8192 one 1024-lane workgroup per CU
// instead of two); with it they fit 64 without spilling.  The XOR layout
// (the comparison option) keeps the compiler's choice: at 64 it spills.
constexpr int bfp_min_waves(int v, int layout) { return (v == 8 && layout != LAYOUT_XOR) ? 8 : 1; }

// The BFP kernels take the per-exchange layouts at every plan: under the
// 64-VGPR bound above the radix-8 N = 8192 plan fits them without spilling
// (the fp32 kernel of that plan does not, so it keeps the padded layout).
constexpr int bfp_lds_layout(int n, int v) { return (void)n, (void)v, LAYOUT_XCHG; }

// The kernel body; BPERM: the filter in the reference's bperm layout, a
// kernel of its own so that the digit-order and pair kernels carry no code
// for it.
template<int N, int V, int LAYOUT, int MID, bool BIG, bool BPERM>
__device__ __forceinline__ void bfp_body(const BfpParams& p)
{
   using PL = Plan<N, V>;
   using LD = Lds<V, LAYOUT>;
   constexpr int T     = PL::T;
   constexpr int CPB   = bfp_cpb(T);
   constexpr int SLOT  = LD::size(N);
   static_assert(T >= 64, "a wavefront register must lie inside one block");

   extern __shared__ float2 lds[];
   const int slot = threadIdx.x / T;
   const int L    = threadIdx.x % T;
   const int lane = threadIdx.x & 63;
   const uint32_t t = blockIdx.x * CPB + slot;    // uniform per wavefront (T >= 64)
   if(t >= p.ntrans) return;
   const uint32_t tu = (uint32_t)uniform((int)t);
   const int w = uniform(L >> 6);                 // wavefront within the transform
   const int lb = BIG ? p.log_block : 6;          // log2 of the block length
   const int nbk = N >> lb;                       // exponent blocks per transform
   // block of (wavefront w, register q): its first point is 64*w + q*T
   auto block_of = [&](int q) { return BIG ? (64 * w + q * T) >> lb : w + q * (T / 64); };

   float2* A = lds + slot * SLOT;
   // per-block abs-max bits (B > 64 only), after the exchange slots; zeroed
   // here, ordered before the atomics by the exchanges' barriers (or, for a
   // transform inside one wavefront, by program order)
   uint32_t* bmax = reinterpret_cast<uint32_t*>(lds + CPB * SLOT) + slot * bfp_bmax_words(N);
   if constexpr(BIG) {
      if(L < nbk) bmax[L] = 0u;
   }
   Twiddles<PL> tw;
   tw.load(p.tw, L);

   // this wavefront's V input exponents.  B = 64: the address is uniform and
   // nothing in the kernel has stored yet, so these are scalar loads (aligned
   // dwords of the transform's N/64 exponent bytes, a multiple of 4; the array
   // is 4-byte aligned by the entry point's contract) and the bytes are picked
   // apart in SALU.  B > 64: a transform's exponents need not fill whole
   // dwords, so lane l reads register l % V's byte through a bounds-checked
   // buffer load and the registers take it by readlane.
   const size_t ebase = (size_t)tu * nbk;
   const uint32_t* ew = reinterpret_cast<const uint32_t*>(p.ein + (BIG ? 0 : ebase));
   int ein_lane = 0;
   if constexpr(BIG) {
      const Buf eb(p.ein + ebase, (uint32_t)nbk);
      ein_lane = eb.ldi8((uint32_t)block_of(lane % V), 0);
   }

   const Buf qb(static_cast<const char*>(p.qin) + (size_t)tu * N * 4, N * 4);
   auto exponent = [&](int q) {
      if constexpr(BIG) {
         return __builtin_amdgcn_readlane(ein_lane, q);
      } else {
         const int byte = block_of(q);
         return (int)(int8_t)(ew[byte >> 2] >> (8 * (byte & 3)));
      }
   };
   float2 r[V];
   // Radix 16 at N = 2048 and 4096: every signal load goes out before the
   // first dequantisation (the empty asm reads them all).  Left to itself the
   // scheduler interleaves loads and dequantisation, 5-8 waits among the 16
   // loads.  The exponents are read first: after the asm the compiler no
   // longer proves them unchanged and would read them with vector loads.
   // Same box: N = 2048 399 -> 416 Gpt/s (+4%), N = 4096 397 -> 397 (another
   // box: 377 -> 384); at N = 16384 it costs 3.7% and elsewhere it is even.
   if constexpr(V == 16 && N >= 2048 && N <= 4096) {
      int ex[V];
      uint32_t wd[V];
#pragma unroll
      for(int q = 0; q < V; q++) ex[q] = exponent(q);
#pragma unroll
      for(int q = 0; q < V; q++) wd[q] = qb.ldu<POL_NT>((uint32_t)L * 4u, q * T * 4);
#pragma unroll
      for(int q = 0; q < V; q++) asm volatile("" :: "v"(wd[q]));
#pragma unroll
      for(int q = 0; q < V; q++)
         r[q] = make_float2(__builtin_amdgcn_ldexpf((float)(int)(int16_t)(wd[q] & 0xffffu), ex[q]),
                            __builtin_amdgcn_ldexpf((float)((int)wd[q] >> 16), ex[q]));
   } else {
#pragma unroll
      for(int q = 0; q < V; q++) {
         const uint32_t word = qb.ldu<POL_NT>((uint32_t)L * 4u, q * T * 4);
         const int e = exponent(q);
         r[q] = make_float2(__builtin_amdgcn_ldexpf((float)(int)(int16_t)(word & 0xffffu), e),
                            __builtin_amdgcn_ldexpf((float)((int)word >> 16), e));
      }
   }

   KeptChain<PL> kc;
   forward_dif<PL, LD, (T < 64 ? 64 : T), 64, KEEP_STORE>(r, A, L, tw, kc);
   {
      const Buf fb(p.filt, p.fcount * (uint32_t)N * 8u);
      const uint32_t f0 = modulo_count(t, p.fcount) * N * 8u;
      if constexpr(BPERM)    mid_op<PL, MID>(r, fb, f0 + L * 8u, T * 8u);
      else if(p.fl == FLT_DR) mid_op_pairs<PL, MID>(r, fb, f0 + L * V * 8u, 16u);
      else                    mid_op_pairs<PL, MID>(r, fb, f0 + L * 16u, T * 16u);
   }
   inverse_dit<PL, LD, (T < 64 ? 64 : T), 64, KEEP_USE>(r, A, L, tw, kc);

   // quantise: register q of this wavefront is block w + q*T/64
   uint32_t m[V];
#pragma unroll
   for(int q = 0; q < V; q++)
      m[q] = __builtin_bit_cast(uint32_t, __builtin_fmaxf(__builtin_fabsf(r[q].x), __builtin_fabsf(r[q].y)));
   // lane l: the abs-max of register l % V over the wavefront
   const uint32_t wmax = block_maxima<V>(m, (uint32_t)lane);
   int e_lane;                                    // exponent of register lane % V's block
   if constexpr(BIG) {
      if(lane < V) atomicMax(&bmax[block_of(lane)], wmax);
      if constexpr(T > 64) __syncthreads();       // CPB == 1: every wavefront is this transform's
      else                 pass_barrier<64>();
      e_lane = bfp_exponent_bits(bmax[block_of(lane % V)]);
   } else {
      e_lane = bfp_exponent_bits(wmax);
   }
   const Buf ob(static_cast<char*>(p.qout) + (size_t)tu * N * 4, N * 4);
   int eq[V];
   int emin = 127;
#pragma unroll
   for(int q = 0; q < V; q++) {
      eq[q] = __builtin_amdgcn_readlane(e_lane, q);
      emin = eq[q] < emin ? eq[q] : emin;
   }
   // low halfwords of yr (bytes 0-1) and yi (bytes 4-5 of {yi, yr}) -> {im, re}
   auto store = [&](int q, float yr, float yi) {
      const uint32_t word = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, yi),
                                                  __builtin_bit_cast(uint32_t, yr), 0x05040100u);
      ob.stu<POL_NT>(word, (uint32_t)L * 4u, q * T * 4);
   };
   // Adding 1.5 * 2^23 rounds |v| < 2^22 to the nearest integer, ties to even
   // (= rint), and leaves it in the low mantissa bits.  With the exact scale
   // 2^-e as a float (127 - e in [1, 254]; e is at most 114 for a finite
   // block) one fma does both steps: v * 2^-e is exact, so rounding
   // v * 2^-e + 1.5 * 2^23 once equals rounding ldexp(v, -e) + 1.5 * 2^23 (a
   // product below 2^-126 rounds to q = 0 either way).  e = -128 has no float
   // 2^128: a wavefront with such a block takes the two-step form for all of
   // its registers (the branch is uniform).
   if(emin > -128) {
#pragma unroll
      for(int q = 0; q < V; q++) {
         const float sc = __builtin_bit_cast(float, (uint32_t)(127 - eq[q]) << 23);
         store(q, __builtin_fmaf(r[q].x, sc, 12582912.0f), __builtin_fmaf(r[q].y, sc, 12582912.0f));
      }
   } else {
#pragma unroll
      for(int q = 0; q < V; q++)
         store(q, __builtin_amdgcn_ldexpf(r[q].x, -eq[q]) + 12582912.0f,
               __builtin_amdgcn_ldexpf(r[q].y, -eq[q]) + 12582912.0f);
   }
   // one store per block, by the lane of its first (wavefront, register) pair
   if(lane < V && (!BIG || ((64 * w + lane * T) & ((1 << lb) - 1)) == 0)) {
      const Buf xb(p.eout + ebase, nbk);
      __builtin_amdgcn_raw_buffer_store_b8((unsigned char)e_lane, xb.r, (uint32_t)block_of(lane), 0, 0);
   }
}

template<int N, int V, int LAYOUT, int MID, bool BIG>
__global__ void __launch_bounds__(bfp_cpb(N / V) * (N / V), bfp_min_waves(V, LAYOUT))
bfp_kernel(const BfpParams p)
{
   bfp_body<N, V, LAYOUT, MID, BIG, false>(p);
}

template<int N, int V, int LAYOUT, int MID, bool BIG>
__global__ void __launch_bounds__(bfp_cpb(N / V) * (N / V), bfp_min_waves(V, LAYOUT))
bfp_bperm_kernel(const BfpParams p)
{
   bfp_body<N, V, LAYOUT, MID, BIG, true>(p);
}

template<int N, int V, int LAYOUT, int MID>
static hipError_t launch_bfp_one(const BfpParams& p, hipStream_t s)
{
   constexpr int T = N / V, CPB = bfp_cpb(T);
   const bool big = p.log_block > 6;
   if(p.log_block < 6 || (1 << p.log_block) > N) return hipErrorInvalidValue;
   const size_t shm = (size_t)CPB * Lds<V, LAYOUT>::size(N) * sizeof(float2)
                    + (big ? (size_t)CPB * bfp_bmax_words(N) * 4 : 0);
   const bool bp = mid_reads_filter<MID> && p.fl == FLT_BPERM;
   const void* k = big ? reinterpret_cast<const void*>(&bfp_kernel<N, V, LAYOUT, MID, true>)
                       : reinterpret_cast<const void*>(&bfp_kernel<N, V, LAYOUT, MID, false>);
   // (the XOR layout is a comparison option and has no bperm kernels)
   if constexpr(mid_reads_filter<MID> && LAYOUT != LAYOUT_XOR) {
      if(bp) k = big ? reinterpret_cast<const void*>(&bfp_bperm_kernel<N, V, LAYOUT, MID, true>)
                     : reinterpret_cast<const void*>(&bfp_bperm_kernel<N, V, LAYOUT, MID, false>);
   } else {
      if(bp) return hipErrorInvalidValue;
   }
   if(!modulo_count_ok(p.fcount, p.ntrans)) return hipErrorInvalidValue;
   static std::atomic<uint64_t> lds_ok[4]{};
   if(const hipError_t e = ensure_dynamic_lds(k, shm, lds_ok[2 * bp + big]); e != hipSuccess) return e;
   const dim3 grid((p.ntrans + CPB - 1) / CPB), block(CPB * T);
   BfpParams arg = p;
   void* argv[] = { &arg };
   return hipLaunchKernel(k, grid, block, argv, shm, s);
}

template<int N, int V>
static hipError_t launch_bfp_nv(int layout, const BfpParams& p, hipStream_t s)
{
   if(layout == LAYOUT_XOR)
      return with_mid(p.mid, [&](auto m) { return launch_bfp_one<N, V, LAYOUT_XOR, decltype(m)::value>(p, s); });
   return with_mid(p.mid, [&](auto m) { return launch_bfp_one<N, V, bfp_lds_layout(N, V), decltype(m)::value>(p, s); });
}

// ---- the reference's own format: one fp32 scale per transform -------------------------
// fufft_pipeline_v16_bfp (fufft.cuh:1614-1701) as its CPU transcription
// states it (kernel_v16_bfp, bfp_quantize; verify_kernel.cpp:1092-1135): a
// transform's points are int16 pairs with one fp32 scale, x = q * scale; the
// filter is int16 pairs in digit order with one fp32 scale per filter,
// b = qb * scale_b, multiplied in at the M = 1 boundary; the result's scale is
// mx / 32767 with mx = max(absmax of the transform's fp32 result, 1e-30), and
// q = rint(clamp(v * (32767 / mx), -32767, 32767)).  Between the codecs runs
// the fp32 pipeline of conv1d.hip, so with the reference's base twiddles the
// words and scales are the transcription's bit for bit.  The abs-max is exact
// in any order: a transform's lanes reduce it in registers (DPP and permlane
// moves, the bits of non-negative floats compared as unsigned), and the
// wavefronts of a transform wider than 64 lanes meet in one LDS word.

// maximum over each group of T lanes (T = 16, 32: the lanes of one transform
// inside a wavefront; T >= 64: the whole wavefront), in every lane
template<int T>
__device__ __forceinline__ uint32_t lanes_max(uint32_t x)
{
   static_assert(T >= 16, "a transform fills at least one row of 16 lanes");
   x = umax(x, dpp_u<0xB1>(x));            // quad_perm [1,0,3,2]
   x = umax(x, dpp_u<0x4E>(x));            // quad_perm [2,3,0,1]
   x = umax(x, dpp_u<0x124>(x));           // row_ror:4
   x = umax(x, dpp_u<0x128>(x));           // row_ror:8: the row of 16
   if constexpr(T >= 32) x = swap_max16(x);
   if constexpr(T >= 64) x = swap_max32(x);
   return x;
}

// The lane's V int16 filter words (re | im << 16, digit-order slots L*V + k)
// dequantised by sb, then the mid operation.  Word k sits at voff + 4k in
// digit order (16-byte loads of four words), at voff + (k/2)*8T + 4(k%2)
// lane-major (8-byte loads of a pair; the slots of the fp32 pair layout) and
// at voff + 4kT in the reference's bperm (4-byte loads); voff is the lane's
// first word: 4(f*N + L*V), 4f*N + 8L and 4(f*N + L).  All V words are read
// before the first product: with each 16-byte load feeding its four products
// in turn, radix 16 at N = 8192 ran at 0.92 of the block-format conv's rate
// on the same box, against 1.00 now (the three layouts within 2% of each
// other at every size).
template<class PL, int MID, bool BPERM>
__device__ __forceinline__ void mid_op_i16(float2 (&r)[PL::V], const Buf& fb, uint32_t voff, int fl, float sb)
{
   using Op = MidOf<MID>;
   constexpr int V = PL::V, T = PL::T;
   uint32_t w[V];
   if constexpr(BPERM) {
#pragma unroll
      for(int k = 0; k < V; k++) w[k] = fb.ldu(voff, k * T * 4);
   } else if(fl == FLT_DR) {
#pragma unroll
      for(int m = 0; m < V / 4; m++) {
         const float4 q = fb.ld4(voff, m * 16);
         w[4 * m]     = __builtin_bit_cast(uint32_t, q.x);
         w[4 * m + 1] = __builtin_bit_cast(uint32_t, q.y);
         w[4 * m + 2] = __builtin_bit_cast(uint32_t, q.z);
         w[4 * m + 3] = __builtin_bit_cast(uint32_t, q.w);
      }
   } else {
#pragma unroll
      for(int m = 0; m < V / 2; m++) {
         const float2 q = fb.ld2(voff, m * T * 8);
         w[2 * m]     = __builtin_bit_cast(uint32_t, q.x);
         w[2 * m + 1] = __builtin_bit_cast(uint32_t, q.y);
      }
   }
#pragma unroll
   for(int k = 0; k < V; k++)
      r[k] = Op::apply(r[k], make_float2((float)(int)(int16_t)(w[k] & 0xffffu) * sb, (float)((int)w[k] >> 16) * sb));
}

template<int N, int V, int LAYOUT, int MID, bool BPERM>
__global__ void __launch_bounds__(bfp_cpb(N / V) * (N / V), bfp_min_waves(V, LAYOUT))
bfp_scaled_kernel(const BfpScaledParams p)
{
   using PL = Plan<N, V>;
   using LD = Lds<V, LAYOUT>;
   using Op = MidOf<MID>;
   constexpr int T     = PL::T;
   constexpr int CPB   = bfp_cpb(T);
   constexpr int SLOT  = LD::size(N);
   constexpr int LANES = T < 64 ? 64 : T;
   constexpr int TPW   = T < 64 ? 64 / T : 1;     // transforms per wavefront

   extern __shared__ float2 lds[];
   const int slot = threadIdx.x / T;
   const int L    = threadIdx.x % T;
   const uint32_t t = blockIdx.x * CPB + slot;
   if(t >= p.ntrans) return;                      // T > 64 => CPB == 1: whole group leaves
   // the wavefront's first transform and this lane's point offset from it
   const uint32_t t0 = (T >= 64) ? (uint32_t)uniform((int)t)
                                 : blockIdx.x * CPB + (uint32_t)uniform((int)(threadIdx.x / 64)) * TPW;
   const uint32_t lane_pos = (T >= 64) ? (uint32_t)L : (t - t0) * N + L;
   const uint32_t tu = (T >= 64) ? t0 : t;        // uniform where a wavefront is one transform

   float2* A = lds + slot * SLOT;
   // wavefronts of one transform (T > 64) meet in this word, zeroed here and
   // ordered before the atomics by the exchanges' workgroup barriers
   uint32_t* amax = reinterpret_cast<uint32_t*>(lds + CPB * SLOT);
   if constexpr(T > 64) {
      if(L == 0) amax[0] = 0u;
   }
   Twiddles<PL> tw;
   tw.load(p.tw, L);

   // both scales up front: after the asm below the compiler no longer proves
   // them unchanged and would read them with vector loads
   const float sa = p.sin[tu];
   const uint32_t fi = modulo_count(tu, p.fcount);
   const float sb = Op::reads_filter ? p.sfilt[fi] : 0.0f;
   const Buf qb(static_cast<const char*>(p.qin) + (size_t)t0 * N * 4, TPW * N * 4);
   // every signal load goes out before the first dequantisation (the empty
   // asm reads them all): left to itself the scheduler interleaves loads and
   // multiplies with up to 12 waits among the 16 loads, and radix 16 at
   // N = 1024 / 8192 / 16384 runs 367 / 232 / 229 Gpt/s against 426 / 282 /
   // 262 (same box; other plans even)
   float2 r[V];
   uint32_t wd[V];
#pragma unroll
   for(int q = 0; q < V; q++) wd[q] = qb.ldu<POL_NT>(lane_pos * 4u, q * T * 4);
#pragma unroll
   for(int q = 0; q < V; q++) asm volatile("" :: "v"(wd[q]));
#pragma unroll
   for(int q = 0; q < V; q++)
      r[q] = make_float2((float)(int)(int16_t)(wd[q] & 0xffffu) * sa, (float)((int)wd[q] >> 16) * sa);

   KeptChain<PL> kc;
   forward_dif<PL, LD, LANES, 64, KEEP_STORE>(r, A, L, tw, kc);
   if constexpr(Op::reads_filter) {
      const Buf fb(p.qfilt, p.fcount * (uint32_t)N * 4u);
      const uint32_t f0 = fi * N * 4u;
      const uint32_t lo = BPERM ? (uint32_t)L * 4u : p.fl == FLT_DR ? (uint32_t)L * V * 4u : (uint32_t)L * 8u;
      mid_op_i16<PL, MID, BPERM>(r, fb, f0 + lo, p.fl, sb);
   } else {
#pragma unroll
      for(int k = 0; k < V; k++) r[k] = Op::apply(r[k], make_float2(0.f, 0.f));
   }
   inverse_dit<PL, LD, LANES, 64, KEEP_USE>(r, A, L, tw, kc);

   // the transform's abs-max
   float m = 0.0f;
#pragma unroll
   for(int q = 0; q < V; q++) m = __builtin_fmaxf(m, __builtin_fmaxf(__builtin_fabsf(r[q].x), __builtin_fabsf(r[q].y)));
   uint32_t x = lanes_max<T>(__builtin_bit_cast(uint32_t, m));
   if constexpr(T > 64) {
      if((threadIdx.x & 63) == 0) atomicMax(amax, x);
      __syncthreads();                            // CPB == 1: every wavefront is this transform's
      x = amax[0];
   }
   const float mx  = __builtin_fmaxf(__builtin_bit_cast(float, x), 1e-30f);
   const float inv = 32767.0f / mx;
   // Adding 1.5 * 2^23 to a value of magnitude <= 32767 rounds it to the
   // nearest integer, ties to even, into the low mantissa bits; the low
   // halfwords of re and im make the output word
   const Buf ob(static_cast<char*>(p.qout) + (size_t)t0 * N * 4, TPW * N * 4);
#pragma unroll
   for(int q = 0; q < V; q++) {
      const float yr = __builtin_fminf(__builtin_fmaxf(r[q].x * inv, -32767.0f), 32767.0f) + 12582912.0f;
      const float yi = __builtin_fminf(__builtin_fmaxf(r[q].y * inv, -32767.0f), 32767.0f) + 12582912.0f;
      const uint32_t word = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, yi),
                                                  __builtin_bit_cast(uint32_t, yr), 0x05040100u);
      ob.stu<POL_NT>(word, lane_pos * 4u, q * T * 4);
   }
   if(L == 0) p.sout[t] = mx / 32767.0f;
}

template<int N, int V, int MID>
static hipError_t launch_bfp_scaled_one(const BfpScaledParams& p, hipStream_t s)
{
   constexpr int T = N / V, CPB = bfp_cpb(T);
   constexpr int LAYOUT = bfp_lds_layout(N, V);
   const size_t shm = (size_t)CPB * Lds<V, LAYOUT>::size(N) * sizeof(float2) + (T > 64 ? 4 : 0);
   if(p.fl != FLT_DR && p.fl != FLT_LANE && p.fl != FLT_BPERM) return hipErrorInvalidValue;
   // the bperm reads get a kernel of their own (mids that read the filter only)
   const bool bp = mid_reads_filter<MID> && p.fl == FLT_BPERM;
   const void* k = reinterpret_cast<const void*>(&bfp_scaled_kernel<N, V, LAYOUT, MID, false>);
   if constexpr(mid_reads_filter<MID>) {
      if(bp) k = reinterpret_cast<const void*>(&bfp_scaled_kernel<N, V, LAYOUT, MID, true>);
   }
   if(!modulo_count_ok(p.fcount, p.ntrans)) return hipErrorInvalidValue;
   static std::atomic<uint64_t> lds_ok[2]{};
   if(const hipError_t e = ensure_dynamic_lds(k, shm, lds_ok[bp]); e != hipSuccess) return e;
   const dim3 grid((p.ntrans + CPB - 1) / CPB), block(CPB * T);
   BfpScaledParams arg = p;
   void* argv[] = { &arg };
   return hipLaunchKernel(k, grid, block, argv, shm, s);
}

template<int N, int V>
static hipError_t launch_bfp_scaled_nv(const BfpScaledParams& p, hipStream_t s)
{
   return with_mid(p.mid, [&](auto m) { return launch_bfp_scaled_one<N, V, decltype(m)::value>(p, s); });
}

bool bfp_scaled_supported(int n, int v)
{
   if(v == 8)  return n >= 512 && n <= 8192 && (n & (n - 1)) == 0;
   if(v == 16) return n >= 256 && n <= 16384 && (n & (n - 1)) == 0;
   return false;
}

hipError_t launch_bfp_scaled(int n, int v, const BfpScaledParams& p, hipStream_t s)
{
   if(v == 8) {
      switch(n) {
         case 512:  return launch_bfp_scaled_nv<512, 8>(p, s);
         case 1024: return launch_bfp_scaled_nv<1024, 8>(p, s);
         case 2048: return launch_bfp_scaled_nv<2048, 8>(p, s);
         case 4096: return launch_bfp_scaled_nv<4096, 8>(p, s);
         case 8192: return launch_bfp_scaled_nv<8192, 8>(p, s);
         default:   break;
      }
   } else if(v == 16) {
      switch(n) {
         case 256:   return launch_bfp_scaled_nv<256, 16>(p, s);
         case 512:   return launch_bfp_scaled_nv<512, 16>(p, s);
         case 1024:  return launch_bfp_scaled_nv<1024, 16>(p, s);
         case 2048:  return launch_bfp_scaled_nv<2048, 16>(p, s);
         case 4096:  return launch_bfp_scaled_nv<4096, 16>(p, s);
         case 8192:  return launch_bfp_scaled_nv<8192, 16>(p, s);
         case 16384: return launch_bfp_scaled_nv<16384, 16>(p, s);
         default:    break;
      }
   }
   return hipErrorInvalidValue;
}

bool bfp_supported(int n, int v)
{
   if(v == 8)  return n >= 512 && n <= 8192 && (n & (n - 1)) == 0;
   if(v == 16) return n >= 1024 && n <= 16384 && (n & (n - 1)) == 0;
   return false;
}

hipError_t launch_bfp(int n, int v, int layout, const BfpParams& p, hipStream_t s)
{
   if(v == 8) {
      switch(n) {
         case 512:  return launch_bfp_nv<512, 8>(layout, p, s);
         case 1024: return launch_bfp_nv<1024, 8>(layout, p, s);
         case 2048: return launch_bfp_nv<2048, 8>(layout, p, s);
         case 4096: return launch_bfp_nv<4096, 8>(layout, p, s);
         case 8192: return launch_bfp_nv<8192, 8>(layout, p, s);
         default:   break;
      }
   } else if(v == 16) {
      switch(n) {
         case 1024:  return launch_bfp_nv<1024, 16>(layout, p, s);
         case 2048:  return launch_bfp_nv<2048, 16>(layout, p, s);
         case 4096:  return launch_bfp_nv<4096, 16>(layout, p, s);
         case 8192:  return launch_bfp_nv<8192, 16>(layout, p, s);
         case 16384: return launch_bfp_nv<16384, 16>(layout, p, s);
         default:    break;
      }
   }
   return hipErrorInvalidValue;
}

}  // namespace fufft
