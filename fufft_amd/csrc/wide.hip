// Fused cyclic convolution at N = 32768 in one launch (gfx950).
//
// The reference runs a single-block conv up to N = 4096 and goes four-step
// beyond (run_large, bench_fufft.cu:357-492: 56 bytes per point over HBM).  A
// CU of MI355X holds 512 KiB of VGPRs, so one workgroup of 1024 lanes keeps a
// whole 32768-point transform in registers, 32 values per lane, and the conv
// becomes the radix-16 plan of the single-launch kernels, LEAD 8 then three
// radix-16 passes (the plan fufft_pipeline_v16 would run at this N,
// fufft.cuh:722-800), with each lane doing the work of two radix-16 lanes:
// groups L and L + T of every radix-16 pass (T = 1024 lanes), four groups of
// the radix-8 lead pass.  The arithmetic per group is the radix-16 kernels'
// own (compute_pass, the reference's butterflies and twiddle chains), so the
// result is bit for bit that plan's and the filter is the radix-16 plan's: in
// digit order, lane-major pairs or bperm, as fufft_plan_filter_f32 writes them
// for (32768, FUFFT_V16).  The signal crosses HBM twice (16 bytes per point),
// the filter once per launch when shared.
//
// The exchanges.  A complex exchange of 32768 points needs 256 KiB, beyond
// the CU's 160 KiB of LDS.  Each exchange therefore runs in two rounds through
// one float buffer of N + N/16 slots (136 KiB): every lane writes the real
// parts of its outgoing values, barrier, reads the real parts of its incoming
// ones, barrier, the same for the imaginary parts.  A lane's register keeps
// the component it has not yet exchanged, so no register is spent on staging.
// The slot layouts (Pad16, Pad256 below) keep every access free of bank
// conflicts.
//
// Races.  Within a pass a lane writes the positions it read, so the next
// exchange's first write needs no barrier after the last read: a pass that
// spans wavefronts reads and writes the same layout (the same slots), a pass
// inside each wavefront may switch layouts but stays in its wavefront's own
// slot range (the layouts below).  The three barriers of an exchange separate
// write from read within a round and the two rounds from each other.  Every
// wavefront of the workgroup reaches every barrier (one transform per
// workgroup, the whole group leaves together).
//
// Resources: 128 VGPRs with no scratch (16 wavefronts of 1024 lanes, 4 per
// SIMD), 136 KiB of LDS: one workgroup per CU.  Measured at 2^27 points on one
// MI355X: 199-207 Gpt/s with the lane-major filter, 187-195 with the
// digit-order one, against 135-138 for the four-step chain at the same N (48
// bytes per point over HBM and the Infinity Cache).
//
// N = 16384 runs the same code with 512 lanes (LEAD 4, eight groups per lane
// in the lead pass): 68 KiB of LDS, so two workgroups share a CU and one's
// loads overlap the other's passes.  fufft_conv_f32 takes it for a shared
// lane-major filter (+2.8% over the workgroup kernel, bit-identical).
#include "fufft_device.hpp"
#include "fufft_plan.hpp"
#include "fufft_internal.hpp"

namespace fufft {

namespace {

template<int N>
using WPlan = Plan<N, 32, 16>;

// Float slot layouts.  gfx950 serves the 4-byte LDS forms 32 lanes at a time
// over 32 banks (bank = slot mod 32), each access of a paired form
// (ds_read2_b32, ds_write2st64_b32) like a single one; a group costs the
// largest number of distinct slots sharing a bank, minus one, in cycles
// (measured with a probe: stride 2 / 4 / 16 cost 2 / 6 / 30 cycles per
// wavefront instruction, strides 17 and 33 nothing).
//  - Pad16, i + i/16: 17 slots per lane at M = 1 and 272 per 16 lanes at
//    M = 16, both conflict free; a run of 32 consecutive positions (the
//    M >= 64 passes) spans 34 slots and costs 2 cycles per access, 768 per
//    wavefront over a transform (the counter's reading).
//  - Pad256, i + 16*(i/256): 32-runs stay contiguous, and the M = 16 pass's
//    two 16-runs per half-wavefront land 16 banks apart: conflict free for
//    the passes at M >= 16, not at M = 1.
// Each exchange takes the layout its two passes need (Pad256 for the ones
// between the M >= 16 passes, Pad16 for the private one into M = 1).  Both put
// the 1024-aligned block c of positions inside slots [1088c, 1088c + 1088),
// so a private pass that reads one layout and writes the other stays inside
// its wavefront's own slot range; both are additive over every pass's taps
// (base + k*M).
struct Pad16 {
   __device__ __forceinline__ static int phys(int i) { return i + (i >> 4); }
   static constexpr int cphys(int i) { return i + (i >> 4); }
   static constexpr int size(int n) { return n + n / 16; }
};
struct Pad256 {
   __device__ __forceinline__ static int phys(int i) { return i + ((i >> 8) << 4); }
   static constexpr int cphys(int i) { return i + ((i >> 8) << 4); }
   static constexpr int size(int n) { return n + n / 16; }
};
static_assert(Pad16::size(CONV_WIDE_N) == Pad256::size(CONV_WIDE_N) && Pad16::size(16384) == Pad256::size(16384),
              "one buffer for both layouts");

// one component (C = 0 real, 1 imaginary) of the lane's values out to pass P's
// positions, or in from them
template<class PL, int P, int C, class FL>
__device__ __forceinline__ void scatter_part(const float2 (&r)[PL::V], float* A, int L)
{
   constexpr int R = PL::radix(P), G = PL::V / R, M = PL::stride(P);
#pragma unroll
   for(int g = 0; g < G; g++) {
      const int bp = FL::phys(tap_pos<PL, P>(L, g, 0));
#pragma unroll
      for(int k = 0; k < R; k++) A[bp + FL::cphys(k * M)] = C ? r[g + k * G].y : r[g + k * G].x;
   }
}

template<class PL, int P, int C, class FL>
__device__ __forceinline__ void gather_part(float2 (&r)[PL::V], const float* A, int L)
{
   constexpr int R = PL::radix(P), G = PL::V / R, M = PL::stride(P);
#pragma unroll
   for(int g = 0; g < G; g++) {
      const int bp = FL::phys(tap_pos<PL, P>(L, g, 0));
#pragma unroll
      for(int k = 0; k < R; k++) {
         if constexpr(C) r[g + k * G].y = A[bp + FL::cphys(k * M)];
         else            r[g + k * G].x = A[bp + FL::cphys(k * M)];
      }
   }
}

// An exchange between passes P and P + 1 stays inside each wavefront when
// both run at M <= 64 with the same radix R: for every group g, wavefront w's
// 64 lanes then own positions [(64w + g*T)*R, (64w + g*T + 64)*R) on both
// sides, and the float slots of those positions (a monotonic map) no other
// wavefront's.  Here: the exchange between the last two radix-16 passes (M =
// 16 and 1).  It takes wavefront fences instead of workgroup barriers, 6 of
// the 18 barriers of a transform.
template<class PL, int P>
constexpr bool exchange_private()
{
   return PL::stride(P) <= 64 && PL::stride(P + 1) <= 64 && PL::radix(P) == PL::radix(P + 1);
}

template<bool PRIVATE>
__device__ __forceinline__ void exchange_fence()
{
   if constexpr(PRIVATE) pass_barrier<64>();
   else                  __syncthreads();
}

// pass PS's values out, pass PG's values in: real round, then imaginary round
template<class PL, int PS, int PG>
__device__ __forceinline__ void split_exchange(float2 (&r)[PL::V], float* A, int L)
{
   constexpr bool PRIVATE = exchange_private<PL, (PS < PG ? PS : PG)>();
   using FL = typename std::conditional<PRIVATE, Pad16, Pad256>::type;
   scatter_part<PL, PS, 0, FL>(r, A, L);
   exchange_fence<PRIVATE>();
   gather_part<PL, PG, 0, FL>(r, A, L);
   exchange_fence<PRIVATE>();
   scatter_part<PL, PS, 1, FL>(r, A, L);
   exchange_fence<PRIVATE>();
   gather_part<PL, PG, 1, FL>(r, A, L);
}

// The mid operation.  After the forward DIF register g + 2k of lane L holds
// digit-order slot (L + g*T)*16 + k, i.e. slot 16*L' + k of radix-16 lane
// L' = L + g*T (of T16 = N/16), so the filter is read where the radix-16
// plan's lane L' reads it: 16 contiguous slots in digit order, pairs at
// 2(L' + m*T16) lane-major, slot 16L' + k at L' + k*T16 in bperm.  The layout
// is a template parameter: a run-time branch kept both sides' registers live
// and spilled.
template<class PL, int MID, int FLT>
__device__ __forceinline__ void wide_mid(float2 (&r)[PL::V], const Buf& fb, uint32_t fb0, int L)
{
   using Op = MidOf<MID>;
   constexpr int T = PL::T, G = 2, T16 = PL::N / 16;
#pragma unroll
   for(int g = 0; g < G; g++) {
      const uint32_t l16 = (uint32_t)(L + g * T);
      // at most 4 slots' loads in flight (the empty asm orders each step after
      // the last): all 16 at once pushed the kernel past 128 VGPRs into scratch
      if constexpr(FLT == FLT_BPERM) {
#pragma unroll
         for(int h = 0; h < 16; h += 4) {
            float2 f[4];
#pragma unroll
            for(int k = 0; k < 4; k++) f[k] = fb.ld2((fb0 + l16) * 8u, (h + k) * T16 * 8);
#pragma unroll
            for(int k = 0; k < 4; k++) {
               r[g + G * (h + k)] = Op::apply(r[g + G * (h + k)], f[k]);
               asm volatile("" :: "v"(r[g + G * (h + k)].x));
            }
         }
      } else {
         constexpr bool lane = FLT == FLT_LANE;
         const uint32_t so = lane ? fb0 * 8u + l16 * 16u : (fb0 + l16 * 16u) * 8u;
         constexpr uint32_t ms = lane ? (uint32_t)T16 * 16u : 16u;
#pragma unroll
         for(int h = 0; h < 8; h += 2) {
            float4 q[2];
#pragma unroll
            for(int m = 0; m < 2; m++) q[m] = fb.ld4(so, (h + m) * ms);
#pragma unroll
            for(int m = 0; m < 2; m++) {
               const int a = g + G * (2 * (h + m)), b = g + G * (2 * (h + m) + 1);
               r[a] = Op::apply(r[a], make_float2(q[m].x, q[m].y));
               r[b] = Op::apply(r[b], make_float2(q[m].z, q[m].w));
               asm volatile("" :: "v"(r[a].x), "v"(r[b].x));
            }
         }
      }
   }
}

template<int N_, int MID, int FLT>
__global__ void __launch_bounds__(WPlan<N_>::T, 4)
conv_wide_kernel(const Conv1dParams p)
{
   using PL = WPlan<N_>;
   constexpr int N = PL::N, T = PL::T, V = PL::V;
   extern __shared__ float ldsf[];
   const int L = threadIdx.x;
   const uint32_t t = blockIdx.x;            // one transform per workgroup
   Twiddles<PL> tw;
   tw.load(p.tw, L);
   // the base twiddles held from here (an empty asm that may change them):
   // left free, the scheduler's placement of their loads and uses cost 28-72
   // bytes of scratch per lane; held, the kernel fits 128 VGPRs with none
#pragma unroll
   for(int i = 0; i < Twiddles<PL>::COUNT; i++) asm volatile("" : "+v"(tw.w[i].x), "+v"(tw.w[i].y));
   KeptChain<PL> kc;                         // not kept: two groups per lane
   float2 r[V];
   // the signal read and the result written once: streamed past the caches
   const Buf xb(static_cast<const char*>(p.in0) + (size_t)t * N * 8, N * 8);
#pragma unroll
   for(int q = 0; q < V; q++) r[q] = xb.ld2<POL_NT>((uint32_t)L * 8u, q * T * 8);
   static_for<PL::NP>([&](auto pi) {
      constexpr int P = decltype(pi)::value;
      if constexpr(P > 0) split_exchange<PL, P - 1, P>(r, ldsf, L);
      compute_pass<PL, P, -1, false, KEEP_NONE>(r, tw, kc);
   });
   if constexpr(mid_reads_filter<MID>) {
      const Buf fb(p.filt, p.fcount * (uint32_t)N * 8u);
      wide_mid<PL, MID, FLT>(r, fb, modulo_count(t, p.fcount) * N, L);
   }
   // At N = 16384 the lead pass holds eight groups' base twiddles per lane;
   // read again for the inverse's lead pass (from the cache), they are free
   // in between, and the kernel fits 128 VGPRs with no scratch (48-68 bytes
   // per lane when held throughout).
   constexpr bool RELOAD_LEAD = PL::V / PL::radix(0) > 4;
   static_for<PL::NP>([&](auto qi) {
      constexpr int P = PL::NP - 1 - decltype(qi)::value;
      if constexpr(RELOAD_LEAD && P == 0) {
         tw.template load_pass<0>(Buf(p.tw, FUFFT_TW_ENTRIES * 8u), L);
#pragma unroll
         for(int i = 0; i < PL::V / PL::radix(0); i++) asm volatile("" : "+v"(tw.w[i].x), "+v"(tw.w[i].y));
      }
      compute_pass<PL, P, +1, true, KEEP_NONE>(r, tw, kc);
      if constexpr(P > 0) split_exchange<PL, P, P - 1>(r, ldsf, L);
   });
   const Buf ob(static_cast<char*>(p.out0) + (size_t)t * N * 8, N * 8);
#pragma unroll
   for(int q = 0; q < V; q++) ob.st2<POL_NT>(r[q], (uint32_t)L * 8u, q * T * 8);
}

template<int N, int MID, int FLT>
hipError_t launch_wide_mid(const Conv1dParams& p, hipStream_t s)
{
   const void* k = reinterpret_cast<const void*>(&conv_wide_kernel<N, MID, FLT>);
   constexpr size_t shm = (size_t)Pad16::size(N) * sizeof(float);
   static std::atomic<uint64_t> lds_ok{};
   if(const hipError_t e = ensure_dynamic_lds(k, shm, lds_ok); e != hipSuccess) return e;
   Conv1dParams arg = p;
   void* argv[] = { &arg };
   return hipLaunchKernel(k, dim3(p.ntrans), dim3(WPlan<N>::T), argv, shm, s);
}

}  // namespace

// Per-signal filters address with 32-bit byte offsets: beyond 4 GiB of them
// the launch is split into chunks of transforms (signal, result and filter
// advance together).
template<int N>
hipError_t launch_conv_wide_n(const Conv1dParams& p, hipStream_t s)
{
   if(p.ntrans == 0) return hipSuccess;
   if(!modulo_count_ok(p.fcount, p.ntrans)) return hipErrorInvalidValue;
   if(p.fl != FLT_DR && p.fl != FLT_LANE && p.fl != FLT_BPERM) return hipErrorInvalidValue;
   auto one = [&](const Conv1dParams& q) {
      return with_mid(q.mid, [&](auto m) {
         constexpr int MID = decltype(m)::value;
         if constexpr(!mid_reads_filter<MID>) return launch_wide_mid<N, MID, FLT_DR>(q, s);
         else return q.fl == FLT_LANE ? launch_wide_mid<N, MID, FLT_LANE>(q, s)
                   : q.fl == FLT_BPERM ? launch_wide_mid<N, MID, FLT_BPERM>(q, s) : launch_wide_mid<N, MID, FLT_DR>(q, s);
      });
   };
   constexpr uint64_t bytes = (uint64_t)N * 8;
   if((uint64_t)p.fcount * bytes <= 0xffffffffull) return one(p);
   if(p.fcount != p.ntrans) return hipErrorInvalidValue;
   const uint32_t step = (uint32_t)(0xffffffffull / bytes) & ~255u;
   for(uint32_t t0 = 0; t0 < p.ntrans; t0 += step) {
      Conv1dParams q = p;
      q.ntrans = p.ntrans - t0 < step ? p.ntrans - t0 : step;
      q.fcount = q.ntrans;
      q.in0  = static_cast<const char*>(p.in0) + (size_t)t0 * bytes;
      q.out0 = static_cast<char*>(p.out0) + (size_t)t0 * bytes;
      q.filt = static_cast<const char*>(p.filt) + (size_t)t0 * bytes;
      if(const hipError_t e = one(q); e != hipSuccess) return e;
   }
   return hipSuccess;
}

hipError_t launch_conv_wide(const Conv1dParams& p, int n, hipStream_t s)
{
   if(n == CONV_WIDE_N) return launch_conv_wide_n<CONV_WIDE_N>(p, s);
   if(n == 16384)       return launch_conv_wide_n<16384>(p, s);
   return hipErrorInvalidValue;
}

}  // namespace fufft
