// 1D fused cyclic convolution for gfx950: forward DIF -> mid operation ->
// inverse DIT in one launch, plus the split forward / apply kernels and the
// two-for-one real variant.
//
// Replaces the reference kernels fufft_pipeline_v16 / _v16f / _wide
// (fufft.cuh:1499-1534, 1703-1734), fufft_pipeline_ip / _fused
// (fufft.cuh:1757-1791), fufft_pipeline_fwd / _apply (fufft.cuh:1343-1407) and
// fufft_conv_r2 (fufft.cuh:1273-1330), and the natural-order batched C2C
// fufft_c2c (fufft.cuh:879-904).
//
// Mapping to CDNA4.  A transform of N points is held by T = N/V lanes with V
// values each (V = 16: radix-16 passes; V = 8: radix-8 passes).  T <= 64
// packs 64/T transforms into one wavefront and needs no workgroup barrier at
// all; T > 64 gives one transform per workgroup of T/64 wavefronts.  HBM is
// touched exactly three times per point: the first DIF pass reads the signal
// straight into registers, the mid operation reads the filter in registers at
// the M = 1 boundary, and the last DIT pass writes the result straight from
// registers.  Every other pass boundary is an exchange through LDS.
#include "fufft_device.hpp"
#include "fufft_plan.hpp"
#include "fufft_internal.hpp"


namespace fufft {

constexpr int cpb_for(int T) { return T >= 128 ? 1 : 256 / T; }

// Transform groups one workgroup of the single-launch conv runs in turn.  At
// N = 16384 the transform fills a CU's LDS, one workgroup per CU, and each
// new workgroup starts some 1200 cycles after the last left; eight in a row
// measured 225.3 -> 232.8 and 225.6 -> 230.0 Gpt/s (two boxes, each against
// one per workgroup), the digit-order filter 218.8 -> 223.4.  Elsewhere the
// other resident workgroups hide the start, and the loop cost 3-11%
// (N = 512 .. 8192, 2 to 8 in a row).
// Iterations need no barrier between them: a lane's last LDS reads (the
// inverse's pass-0 gather) and its first LDS writes of the next transform
// (the forward's pass-0 scatter) are the same positions of the same layout,
// which no other lane touches in between.
template<int N, int KIND>
constexpr uint32_t conv_iters() { return (KIND == K_CONV && N == 16384) ? 8u : 1u; }

// A lane's V digit-order values (slots L*V + k of the transform at point
// offset base) as 16-byte pairs: contiguous in digit order, at 2(L + m*T)
// lane-major (FLT_LANE).  One uniform branch; each side computes only its own
// offsets.
template<int V, int T>
__device__ __forceinline__ void store_spectrum(const Buf& ob, const float2 (&r)[V], uint32_t base, int L, int layout)
{
   const bool lane = layout == FLT_LANE;
   const uint32_t so = (base + (lane ? 2u : (uint32_t)V) * (uint32_t)L) * 8u;
   const uint32_t ms = lane ? (uint32_t)T * 16u : 16u;
#pragma unroll
   for(int m = 0; m < V / 2; m++)
      ob.st4(make_float4(r[2 * m].x, r[2 * m].y, r[2 * m + 1].x, r[2 * m + 1].y), so, m * ms);
}

// The kernel body for transform group bid.  BPERM: the filter is in the
// reference's bperm layout (8-byte loads); it gets a kernel of its own so that
// the digit-order and pair kernels carry no code for it.
template<int N, int V, int LAYOUT, int KIND, int MID, bool BPERM>
__device__ __forceinline__ void conv1d_body(const Conv1dParams& p, const uint32_t bid)
{
   using PL = Plan<N, V>;
   using LD = Lds<V, LAYOUT>;
   constexpr int T     = PL::T;
   constexpr int CPB   = cpb_for(T);
   constexpr int SLOT  = LD::size(N);
   constexpr int LANES = T < 64 ? 64 : T;
   constexpr int TPW   = T < 64 ? 64 / T : 1;     // transforms per wavefront
   // bytes per point of the natural-order side in HBM: real pairs x / y (or
   // u / v) travel as two separate float arrays
   constexpr bool REAL_IN   = KIND == K_CONV_R2 || KIND == K_FWD_R2;
   constexpr bool REAL_OUT  = KIND == K_CONV_R2 || KIND == K_APPLY_R2;
   constexpr bool FROM_SPEC = KIND == K_APPLY || KIND == K_APPLY_R2;
   constexpr bool TO_SPEC   = KIND == K_FWD || KIND == K_FWD_R2;
   constexpr bool C2C_FWD   = KIND == K_C2C_FWD;
   constexpr bool C2C_INV   = KIND == K_C2C_INV;
   constexpr bool PLAN      = KIND == K_PLAN_TAPS;
   constexpr bool TIMED     = KIND == K_CONV_TIMED;
   // one filter per signal: its loads go out with the signal's (lane-major
   // pairs, or digit order handed to the lanes through LDS at the mid)
   constexpr bool PSF_ANY   = (KIND == K_CONV_PSF || KIND == K_CONV_PSF_DR) && mid_reads_filter<MID>;
   constexpr bool PSF       = PSF_ANY && (KIND == K_CONV_PSF_DR || conv_psf_plan(N, V));
   constexpr bool PSF_DR    = PSF && KIND == K_CONV_PSF_DR;
   // where the registers allow no early read: the lane-major filter read at
   // the mid as usual, streamed past the caches
   constexpr bool PSF_LATE  = PSF_ANY && !PSF;
   // the signal read and the result written once per launch stream past the
   // caches in the single-launch conv and C2C; the four-step middle, the split
   // and 2D row kernels keep the default policy
   constexpr int  IO_POL    = (KIND == K_CONV || KIND == K_CONV_PSF || KIND == K_CONV_PSF_DR || TIMED || C2C_FWD ||
                               C2C_INV) ? POL_NT
                                                                                              : POL_DEFAULT;
   constexpr int  EL_IN     = REAL_IN ? 4 : 8;
   constexpr int  EL_OUT    = REAL_OUT ? 4 : 8;

   extern __shared__ float2 lds[];
   const int slot = threadIdx.x / T;
   const int L    = threadIdx.x % T;
   const uint32_t t = bid * CPB + slot;
   if(t >= p.ntrans) return;                 // T > 64 => CPB == 1: whole group leaves

   // the wavefront's first transform (uniform) and this lane's offset from it
   const uint32_t t0 = (T >= 64) ? (uint32_t)uniform((int)t)
                                 : bid * CPB + (uint32_t)uniform((int)(threadIdx.x / 64)) * TPW;
   const uint32_t lane_pos = (T >= 64) ? (uint32_t)L : (t - t0) * N + L;

   float2* A = lds + slot * SLOT;
   // phase timer: every memory operation retired and every wavefront of the
   // workgroup arrived, then the shader clock (reads only; thread 0 writes the
   // record with ordinary vector stores at the end)
   uint64_t ts[TIMER_MARKS + 1], rt0 = 0;
   auto stamp = [&](int i) {
      if constexpr(TIMED) {
         __builtin_amdgcn_s_waitcnt(0);
         __syncthreads();
         ts[i] = __builtin_amdgcn_s_memtime();
      }
   };
   stamp(0);
   if constexpr(TIMED) rt0 = __builtin_amdgcn_s_memrealtime();
   Twiddles<PL> tw;
   tw.load(p.tw, L);
   // both halves in this launch: the forward's last twiddled chain serves the inverse
   constexpr int KEEP_F = (KIND == K_CONV || KIND == K_CONV_MID || KIND == K_CONV_R2 || TIMED || PSF_LATE) ? KEEP_STORE
                                                                                                      : KEEP_NONE;
   constexpr int KEEP_I = KEEP_F == KEEP_STORE ? KEEP_USE : KEEP_NONE;
   KeptChain<PL> kc;
   float2 r[V];
   float4 pf[PSF ? V / 2 : 1];

   if constexpr(FROM_SPEC) {
      const Buf sb(p.spec, p.scount * (uint32_t)N * 8u);
      if(p.sl == FLT_LANE) {
         // lane-major pairs: slots L*V + 2m, 2m + 1 at 2(L + m*T), one
         // contiguous KiB per 16-byte load of a wavefront
         const uint32_t so = modulo_count(t, p.scount) * N * 8u + L * 16u;
#pragma unroll
         for(int m = 0; m < V / 2; m++) {
            const float4 q = sb.ld4(so, m * T * 16);
            r[2 * m] = make_float2(q.x, q.y);
            r[2 * m + 1] = make_float2(q.z, q.w);
         }
      } else if constexpr(V == 16 && N >= 2048) {
         // digit order at radix 16: each wavefront's 64 * 16 slots are
         // contiguous, loaded in 1 KiB runs and handed to its lanes through
         // LDS (as the filter read below); read in place every 16-byte load
         // of a wavefront touches 64 cache lines.  Same box, 2^27 points,
         // bit-identical: N = 2048 336 -> 369, 8192 312 -> 342 Gpt/s, 4096
         // even (339).  The LDS reads complete before the filter read reuses
         // the same positions (wavefront fence)
         load_dr_staged<PL, typename LD::template at<PL, PL::NP - 2>>(r, sb, modulo_count(t, p.scount) * N, A, L);
         pass_barrier<64>();
      } else {
         // digit order: slots L*V .. L*V+V-1, two complex per 16-byte load
         const uint32_t so = (modulo_count(t, p.scount) * N + L * V) * 8u;
#pragma unroll
         for(int m = 0; m < V / 2; m++) {
            const float4 q = sb.ld4(so, m * 16);
            r[2 * m] = make_float2(q.x, q.y);
            r[2 * m + 1] = make_float2(q.z, q.w);
         }
      }
      // Radix 8 (8 wavefronts per SIMD): the filter loads of the mid operation
      // wait until the spectrum has arrived (the empty asm reads every value).
      // Issued together with the spectrum loads they cost 3% at N = 4096 (358
      // against 370 Gpt/s, same box); at radix 16 (4 wavefronts per SIMD) the
      // wait costs up to 6% (N = 1024: 304 against 322).
      if constexpr(V == 8) {
#pragma unroll
         for(int k = 0; k < V; k++) asm volatile("" :: "v"(r[k].x), "v"(r[k].y));
      }
   } else {
      const size_t wb = (size_t)t0 * N * EL_IN;
      constexpr uint32_t WB = TPW * N * EL_IN;
      if constexpr(REAL_IN) {
         const Buf xb(static_cast<const char*>(p.in0) + wb, WB);
         const Buf yb(static_cast<const char*>(p.in1) + wb, WB);
#pragma unroll
         for(int q = 0; q < V; q++)
            r[q] = make_float2(xb.ld1(lane_pos * 4u, q * T * 4), yb.ld1(lane_pos * 4u, q * T * 4));
      } else {
         const Buf xb(static_cast<const char*>(p.in0) + wb, WB);
#pragma unroll
         for(int q = 0; q < V; q++) r[q] = xb.ld2<IO_POL>(lane_pos * 8u, q * T * 8);
      }
      if constexpr(PSF) {
         // each signal's own filter is a third stream from HBM: issued here,
         // its latency hides behind the forward DIF instead of the mid phase.
         // N = 4096, one filter per signal, same box: 234.0 / 234.5 -> 243.4 /
         // 243.7 Gpt/s (+4%, bit-identical); at N = 1024 / 2048 +0.7% / even,
         // and with a shared (cache-resident) filter -0.4% for the kept chain
         // it gives up, so it is this plan's per-signal kernel only.  Each
         // filter is read once: NT, as the signal (a property of this kernel,
         // no runtime choice): bit-identical, +1.5% in bench.py's per-signal
         // leg and +3.2% in 100-launch rounds, same box
         const Buf fb(p.filt, p.fcount * (uint32_t)N * 8u);
         if constexpr(PSF_DR) {
            dr_runs_load<PL, POL_NT>(pf, fb, modulo_count(t, p.fcount) * N, L);
         } else {
            const uint32_t so = modulo_count(t, p.fcount) * N * 8u + L * 16u;
#pragma unroll
            for(int m = 0; m < V / 2; m++) pf[m] = fb.ld4<POL_NT>(so, m * T * 16);
         }
      }
      stamp(1);
      if constexpr(C2C_INV) natural_to_digit<PL, LD, LANES, true>(r, A, L);
      else                  forward_dif<PL, LD, LANES, 64, KEEP_F>(r, A, L, tw, kc);
      stamp(2);
   }

   if constexpr(C2C_FWD) {
      digit_to_natural<PL, LD, LANES>(r, A, L);
      const Buf ob(static_cast<char*>(p.out0) + (size_t)t0 * N * 8, TPW * N * 8);
#pragma unroll
      for(int q = 0; q < V; q++) ob.st2<IO_POL>(r[q], lane_pos * 8u, q * T * 8);
      return;
   } else if constexpr(PLAN) {
      const Buf ob(static_cast<char*>(p.out0) + (size_t)t0 * N * 8, TPW * N * 8);
#pragma unroll
      for(int k = 0; k < V; k++) r[k] = make_float2(r[k].x * p.scale, r[k].y * p.scale);
      if(p.fl == FLT_BPERM) {
#pragma unroll
         for(int k = 0; k < V; k++) ob.st2(r[k], lane_pos * 8u, k * T * 8);
      } else {
         store_spectrum<V, T>(ob, r, (t - t0) * N, L, p.fl);
      }
      return;
   } else if constexpr(TO_SPEC) {
      const Buf ob(static_cast<char*>(p.out0) + (size_t)t0 * N * 8, TPW * N * 8);
      // lane-major: every store of a wavefront is one contiguous run.  The
      // digit-order store writes 16 bytes per lane 64 or 128 bytes apart (32
      // or 64 cache lines per wavefront store) and runs 14-18% slower.
      store_spectrum<V, T>(ob, r, (t - t0) * N, L, p.sl);
      return;
   } else {
      if constexpr(!C2C_INV) {
         const Buf fb(p.filt, p.fcount * (uint32_t)N * 8u);
         const uint32_t fb0 = modulo_count(t, p.fcount) * N;
         // a uniform branch on the filter layout: each side computes only its own offset
         if constexpr(PSF_DR) {
            using Op = MidOf<MID>;
            float2 b[V];
            dr_runs_stage<PL, typename LD::template at<PL, PL::NP - 2>>(b, pf, A, L);
#pragma unroll
            for(int k = 0; k < V; k++) r[k] = Op::apply(r[k], b[k]);
         } else if constexpr(PSF) {
            using Op = MidOf<MID>;
#pragma unroll
            for(int m = 0; m < V / 2; m++) {
               r[2 * m]     = Op::apply(r[2 * m], make_float2(pf[m].x, pf[m].y));
               r[2 * m + 1] = Op::apply(r[2 * m + 1], make_float2(pf[m].z, pf[m].w));
            }
         }
         else if constexpr(PSF_LATE) mid_op_pairs<PL, MID, POL_NT>(r, fb, fb0 * 8u + L * 16u, T * 16u);
         else if constexpr(BPERM) mid_op<PL, MID>(r, fb, (fb0 + L) * 8u, T * 8u);
         else if(p.fl == FLT_DR) {
            // radix 16 from N = 2048 (the reference's own plan and filter
            // order): through LDS, N = 2048 / 4096 / 8192 334 -> 348, 312 ->
            // 328, 255 -> 273 Gpt/s (same box); at N = 1024 it cost 2%, at
            // radix 8 2-5% (33% at N = 8192, where it took the workgroups per
            // CU down), and in the BFP conv, VALU-bound, 0 to -11%
            if constexpr(V == 16 && N >= 2048 && mid_reads_filter<MID>)
               mid_op_dr_staged<PL, typename LD::template at<PL, PL::NP - 2>, MID>(r, fb, fb0, A, L);
            else
               mid_op_pairs<PL, MID>(r, fb, (fb0 + L * V) * 8u, 16u);
         }
         else                    mid_op_pairs<PL, MID>(r, fb, fb0 * 8u + L * 16u, T * 16u);
      }
      stamp(3);
      inverse_dit<PL, LD, LANES, 64, KEEP_I>(r, A, L, tw, kc);
      stamp(4);

      const size_t wb = (size_t)t0 * N * EL_OUT;
      constexpr uint32_t WB = TPW * N * EL_OUT;
      if constexpr(REAL_OUT) {
         const Buf ub(static_cast<char*>(p.out0) + wb, WB);
         const Buf vb(static_cast<char*>(p.out1) + wb, WB);
#pragma unroll
         for(int q = 0; q < V; q++) {
            ub.st1(r[q].x, lane_pos * 4u, q * T * 4);
            vb.st1(r[q].y, lane_pos * 4u, q * T * 4);
         }
      } else {
         const Buf ob(static_cast<char*>(p.out0) + wb, WB);
#pragma unroll
         for(int q = 0; q < V; q++) ob.st2<IO_POL>(r[q], lane_pos * 8u, q * T * 8);
      }
      if constexpr(TIMED) {
         stamp(5);
         const uint64_t rt1 = __builtin_amdgcn_s_memrealtime();
         if(threadIdx.x == 0 && blockIdx.x < p.timing_groups) {
            uint32_t* rec = p.timing + (size_t)blockIdx.x * TIMER_STRIDE;
            rec[0] = __builtin_amdgcn_s_getreg((31 << 11) | 4);     // HW_REG_HW_ID
            rec[1] = __builtin_amdgcn_s_getreg((31 << 11) | 20);    // HW_REG_XCC_ID
            rec[2] = TIMER_MARKS;
            rec[3] = (uint32_t)(rt1 - rt0);    // constant 100 MHz clock across the marks
            rec[4] = (uint32_t)ts[0];
            rec[5] = (uint32_t)(ts[0] >> 32);
#pragma unroll
            for(int i = 1; i <= TIMER_MARKS; i++) {
               const uint64_t d = ts[i] - ts[0];
               rec[5 + i] = ((uint32_t)i << 24) | (uint32_t)(d > 0xffffffull ? 0xffffffull : d);
            }
            rec[11] = 0;
         }
      }
   }
}

template<int N, int V, int LAYOUT, int KIND, int MID>
__global__ void __launch_bounds__(cpb_for(N / V) * (N / V))
conv1d_kernel(const Conv1dParams p)
{
   constexpr uint32_t IT = conv_iters<N, KIND>();
#pragma unroll 1
   for(uint32_t it = 0; it < IT; it++) conv1d_body<N, V, LAYOUT, KIND, MID, false>(p, blockIdx.x * IT + it);
}

// the calls that read a filter, with a bperm filter
template<int N, int V, int LAYOUT, int KIND, int MID>
__global__ void __launch_bounds__(cpb_for(N / V) * (N / V))
conv1d_bperm_kernel(const Conv1dParams p)
{
   constexpr uint32_t IT = conv_iters<N, KIND>();
#pragma unroll 1
   for(uint32_t it = 0; it < IT; it++) conv1d_body<N, V, LAYOUT, KIND, MID, true>(p, blockIdx.x * IT + it);
}

// (the XOR layout is a comparison option and has no bperm kernels)
template<int LAYOUT, int KIND, int MID>
constexpr bool reads_bperm_filter()
{
   return LAYOUT != LAYOUT_XOR && mid_reads_filter<MID> &&
          (KIND == K_CONV || KIND == K_CONV_TIMED || KIND == K_CONV_R2 || KIND == K_APPLY);
}

template<int N, int V, int LAYOUT, int KIND, int MID>
static hipError_t launch_one(const Conv1dParams& p, hipStream_t s)
{
   constexpr int T = N / V, CPB = cpb_for(T);
   const size_t shm = (size_t)CPB * Lds<V, LAYOUT>::size(N) * sizeof(float2);
   bool bp = false;
   const void* k = reinterpret_cast<const void*>(&conv1d_kernel<N, V, LAYOUT, KIND, MID>);
   if constexpr(reads_bperm_filter<LAYOUT, KIND, MID>()) {
      if(p.fl == FLT_BPERM) {
         bp = true;
         k = reinterpret_cast<const void*>(&conv1d_bperm_kernel<N, V, LAYOUT, KIND, MID>);
      }
   } else {
      if(mid_reads_filter<MID> && p.fl == FLT_BPERM) return hipErrorInvalidValue;
   }
   if(!modulo_count_ok(p.fcount, p.ntrans) || !modulo_count_ok(p.scount, p.ntrans)) return hipErrorInvalidValue;
   static std::atomic<uint64_t> lds_ok[2]{};
   if(const hipError_t e = ensure_dynamic_lds(k, shm, lds_ok[bp]); e != hipSuccess) return e;
   constexpr uint32_t IT = conv_iters<N, KIND>();
   const dim3 grid((uint32_t)(((uint64_t)p.ntrans + CPB * IT - 1) / (CPB * IT))), block(CPB * T);
   Conv1dParams arg = p;
   void* argv[] = { &arg };
   return hipLaunchKernel(k, grid, block, argv, shm, s);
}

template<int N, int V, int LAYOUT, int KIND>
static hipError_t launch_mid(const Conv1dParams& p, hipStream_t s)
{
   return with_mid(p.mid, [&](auto m) { return launch_one<N, V, LAYOUT, KIND, decltype(m)::value>(p, s); });
}

template<int N, int V, int LAYOUT>
static hipError_t launch_kind(int kind, const Conv1dParams& p, hipStream_t s)
{
   switch(kind) {
      case K_CONV:    return launch_mid<N, V, LAYOUT, K_CONV>(p, s);
      case K_CONV_PSF:
         // lane-major filters only, default LDS layouts (the launcher's choice)
         if constexpr((conv_psf_plan(N, V) || conv_psf_late_plan(N, V)) && LAYOUT != LAYOUT_XOR) {
            return p.fl == FLT_LANE ? launch_mid<N, V, LAYOUT, K_CONV_PSF>(p, s) : hipErrorInvalidValue;
         } else {
            return hipErrorInvalidValue;
         }
      case K_CONV_PSF_DR:
         // digit-order filters only, default LDS layouts (the launcher's choice)
         if constexpr(conv_psf_dr_plan(N, V) && LAYOUT != LAYOUT_XOR) {
            return p.fl == FLT_DR ? launch_mid<N, V, LAYOUT, K_CONV_PSF_DR>(p, s) : hipErrorInvalidValue;
         } else {
            return hipErrorInvalidValue;
         }
      case K_CONV_MID:
         // the four-step middle: N = 512 .. 4096, radix 16 (the reference's
         // middle) or radix 8
         if constexpr(N >= 512 && N <= 4096) return launch_mid<N, V, LAYOUT, K_CONV_MID>(p, s);
         else                                return hipErrorInvalidValue;
      case K_CONV_R2: return launch_one<N, V, LAYOUT, K_CONV_R2, MID_MUL>(p, s);
      case K_FWD:     return launch_one<N, V, LAYOUT, K_FWD, MID_NONE>(p, s);
      case K_APPLY:   return launch_mid<N, V, LAYOUT, K_APPLY>(p, s);
      case K_FWD_R2:  return launch_one<N, V, LAYOUT, K_FWD_R2, MID_NONE>(p, s);
      case K_APPLY_R2:
         // only the 2D two-for-one path uses it, as the row inverse
         return p.mid == MID_NONE ? launch_one<N, V, LAYOUT, K_APPLY_R2, MID_NONE>(p, s)
                                  : hipErrorInvalidValue;
      case K_C2C_FWD:   return launch_one<N, V, LAYOUT, K_C2C_FWD, MID_NONE>(p, s);
      case K_C2C_INV:   return launch_one<N, V, LAYOUT, K_C2C_INV, MID_NONE>(p, s);
      case K_PLAN_TAPS: return launch_one<N, V, LAYOUT, K_PLAN_TAPS, MID_NONE>(p, s);
      case K_CONV_TIMED:
         // the timed build exists for the default LDS layout only
         if constexpr(LAYOUT == default_lds_layout(N, V)) {
            return launch_mid<N, V, LAYOUT, K_CONV_TIMED>(p, s);
         } else {
            return hipErrorInvalidValue;
         }
      default:        return hipErrorInvalidValue;
   }
}

template<int N, int V>
static hipError_t launch_nv(int kind, int layout, const Conv1dParams& p, hipStream_t s)
{
   return layout == LAYOUT_XOR ? launch_kind<N, V, LAYOUT_XOR>(kind, p, s)
                               : launch_kind<N, V, default_lds_layout(N, V)>(kind, p, s);
}

bool conv1d_supported(int n, int v)
{
   if(v == 16) return n >= 256 && n <= 16384 && (n & (n - 1)) == 0;
   if(v == 8)  return n >= 512 && n <= 8192 && (n & (n - 1)) == 0;
   return false;
}

hipError_t launch_conv1d(int kind, int n, int v, int layout, const Conv1dParams& p, hipStream_t s)
{
   if(v == 16) {
      switch(n) {
         case 256:   return launch_nv<256, 16>(kind, layout, p, s);
         case 512:   return launch_nv<512, 16>(kind, layout, p, s);
         case 1024:  return launch_nv<1024, 16>(kind, layout, p, s);
         case 2048:  return launch_nv<2048, 16>(kind, layout, p, s);
         case 4096:  return launch_nv<4096, 16>(kind, layout, p, s);
         case 8192:  return launch_nv<8192, 16>(kind, layout, p, s);
         case 16384: return launch_nv<16384, 16>(kind, layout, p, s);
         default:    break;
      }
   } else if(v == 8) {
      switch(n) {
         case 512:  return launch_nv<512, 8>(kind, layout, p, s);
         case 1024: return launch_nv<1024, 8>(kind, layout, p, s);
         case 2048: return launch_nv<2048, 8>(kind, layout, p, s);
         case 4096: return launch_nv<4096, 8>(kind, layout, p, s);
         case 8192: return launch_nv<8192, 8>(kind, layout, p, s);
         default:   break;
      }
   }
   return hipErrorInvalidValue;
}

}  // namespace fufft
