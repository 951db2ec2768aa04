// Compile-time pass plan and LDS layouts shared by the 1D, BFP and 2D kernels.
//
// A transform of N = LEAD * RM^NR points is held by T = N/V lanes, V values
// per lane, main radix RM = V (or V/2: the 32-values-per-lane conv, whose lanes
// each run two radix-16 groups).  DIF pass p has radix R_p (LEAD first when
// LEAD > 1, then RM) and stride M_p = N / (R_0 ... R_p); DIT runs the same
// passes in reverse.  In pass p lane L owns the G = V/R groups gidx = L + g*T,
// j = gidx % M, b = gidx / M, whose taps sit at b*R*M + j + k*M
// (fufft.cuh:722-756); tap k of group g lives in register g + k*G.  With that
// convention:
//   - pass 0 reads position L + q*T into register q, so the first DIF pass
//     loads straight from HBM and the last DIT pass stores straight to HBM
//     (coalesced across lanes for every q);
//   - the last DIF pass and the first DIT pass run at M = 1 with lane L owning
//     positions L*V .. L*V + V-1 in registers (with two groups per lane,
//     (L + g*T)*RM + k in register g + 2k), so the pointwise mid operation
//     happens in registers between them (fufft.cuh:1435-1443);
//   - every other pass boundary is one exchange through LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>
#include <utility>

#include "fufft_device.hpp"

namespace fufft {

constexpr int ilog2c(int x) { int r = 0; while((1 << r) < x) r++; return r; }

// RM is the radix of the main passes, V by default; with V = 2 * RM every lane
// runs two groups of each main pass (the 32-values-per-lane conv, wide.hip).
template<int N_, int V_, int RM_ = V_>
struct Plan {
   static constexpr int N = N_, V = V_, RM = RM_;
   static constexpr int LOGN = ilog2c(N), LOGV = ilog2c(V), LOGR = ilog2c(RM);
   static constexpr int NR   = LOGN / LOGR;
   static constexpr int LEAD = 1 << (LOGN % LOGR);
   static constexpr int NP   = NR + (LEAD > 1 ? 1 : 0);
   static constexpr int T    = N / V;
   static_assert((1 << LOGN) == N && (1 << LOGV) == V && (1 << LOGR) == RM, "power-of-two sizes only");
   static_assert(NR >= 1, "N must hold at least one main pass");
   static_assert(V % RM == 0 && V % LEAD == 0, "whole groups per lane");

   static constexpr int radix(int p) { return (LEAD > 1 && p == 0) ? LEAD : RM; }
   static constexpr int stride(int p)
   {
      int M = N;
      for(int i = 0; i <= p; i++) M /= radix(i);
      return M;
   }
};

// ---- compile-time loop --------------------------------------------------------
template<class F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>)
{
   (f(std::integral_constant<int, Is>{}), ...);
}
template<int COUNT, class F>
__device__ __forceinline__ void static_for(F&& f)
{
   static_for_impl(f, std::make_integer_sequence<int, COUNT>{});
}

// ---- LDS layouts ------------------------------------------------------------------
// phys(i) maps logical position i of a transform to its float2 slot.  gfx950
// LDS bank model, measured with SQ_LDS_BANK_CONFLICT on a one-off probe kernel
// (restated with the measurements in tests/lds_bank_model.py):
// ds_read_b64 is serviced 32 lanes at a time, so lanes of an aligned
// half-wavefront conflict when their slots agree modulo 32; ds_write_b64 and
// each 8-byte access of the paired forms the exchanges compile to
// (ds_read2_b64, ds_write2_b64, ds_read2st64_b64) are serviced 16 lanes at a
// time, so lanes of an aligned quarter-wavefront conflict when their slots
// agree modulo 16.  Each extra way costs one cycle.  tests/test_lds_audit.py
// checks every access pattern of every plan against both rules.
//
// Xor: bits [0, v) ^= bits [v, 2v), bits [v, 5) ^= bits [2v, v+5).  Conflict
// free for every pass pattern, but the XOR keeps one address register per tap.
// Pad: one spare slot after every V (phys = i + i/V, i.e. 1/16 or 1/8 more
// LDS).  For every pass the padded address is additive,
//    phys(base + k*M) = phys(base) + phys(k*M),
// so a lane computes one address per group and the taps use immediate
// offsets.  At most 2-way conflicts remain in the consecutive-lane passes.
enum { LAYOUT_XOR = 0, LAYOUT_PAD = 1, LAYOUT_XCHG = 2 };
// run-time selection passed to the launchers: each plan's default, or XOR
enum { LAYOUT_DEFAULT = 3 };

template<int V, int LAYOUT>
struct Lds;

// Exchange E (between pass E and pass E + 1) of plan PL: one spare block of
// Mb slots after every Ma = V*Mb positions, phys = i + Mb*(i / Ma), where Mb
// is the stride of the first wavefront-private pass after the exchange (the
// first pass from E + 1 on with M <= 64).
//  - Conflicts: a private reader (M = Mb) reads runs of Mb consecutive
//    positions Ma apart, which land Ma + Mb slots apart and tile the 64 banks;
//    every other pass writes or reads runs of 32 consecutive positions,
//    which no spare block splits.
//  - Additive for both passes' taps: base + k*M never crosses an Ma block in
//    a pass with M <= Mb and crosses k whole blocks in a pass with M >= Ma.
//  - Races: a pass gathers from exchange E-1 and scatters into exchange E
//    with no barrier in between.  A pass that spans wavefronts (M > 64)
//    therefore gets the same layout on both sides (it reads and writes the
//    same slots, as with a single layout); a private pass keeps each
//    wavefront inside its own block of V*64 positions, and both of its
//    layouts map block boundaries to the same slot, so wavefronts never touch
//    each other's slots.
// tests/test_lds_audit.py checks all of this by brute force for every plan.
// Under both rules every exchange is conflict free, where the single padded
// layout below leaves 2-way conflicts after the wide passes.
template<class PL, int E>
struct XchgLds {
   static constexpr int reader_stride(int e)
   {
      int q = e + 1;
      while(PL::stride(q) > 64) q++;
      return PL::stride(q);
   }
   static constexpr int Mb = reader_stride(E), Ma = PL::V * Mb;
   static constexpr bool additive = true;
   __device__ __forceinline__ static int phys(int i) { return i + Mb * (i / Ma); }
   static constexpr int cphys(int i) { return i + Mb * (i / Ma); }
};

// The default layout of a plan: per-exchange (XchgLds) wherever it keeps the
// kernel's VGPRs; at radix 8, N = 8192 its extra exchange base addresses take
// the kernel from 62 to 71 VGPRs, which halves the workgroups per CU, so that
// plan keeps the single padded layout.
constexpr int default_lds_layout(int n, int v) { return (v == 8 && n > 4096) ? LAYOUT_PAD : LAYOUT_XCHG; }

template<int V>
struct Lds<V, LAYOUT_XOR> {
   static constexpr int LOGV = ilog2c(V);
   static constexpr int HI   = 5 - LOGV;      // bits folded into [v, 5)
   static constexpr bool additive = false;
   static constexpr int size(int n) { return n; }
   __device__ __forceinline__ static int phys(int i)
   {
      return i ^ ((i >> LOGV) & (V - 1)) ^ (((i >> (2 * LOGV)) & ((1 << HI) - 1)) << LOGV);
   }
   static constexpr int cphys(int i) { return i; }
   template<class PL, int E> using at = Lds;
};

template<int V>
struct Lds<V, LAYOUT_PAD> {
   static constexpr bool additive = true;
   static constexpr int size(int n) { return n + n / V; }
   __device__ __forceinline__ static int phys(int i) { return i + i / V; }
   static constexpr int cphys(int i) { return i + i / V; }
   template<class PL, int E> using at = Lds;
};

// Per-exchange layouts for the pass exchanges (XchgLds, at most N + N/V
// slots: M_{E+1} / M_E = 1/V for every E); the padded layout for any other
// exchange through the slot (the natural-order C2C's).
template<int V>
struct Lds<V, LAYOUT_XCHG> : Lds<V, LAYOUT_PAD> {
   template<class PL, int E> using at = XchgLds<PL, E>;
};

// ---- pass machinery ---------------------------------------------------------------
template<class PL, int P>
__device__ __forceinline__ int tap_pos(int L, int g, int k)
{
   constexpr int R = PL::radix(P), M = PL::stride(P), T = PL::T;
   const int gidx = L + g * T;
   const int j = gidx & (M - 1), b = gidx / M;
   return b * R * M + j + k * M;
}

// LDS slot of tap k of group g: one address per group plus a compile-time
// offset for additive layouts, the full map per tap otherwise
template<class PL, int P, class LD>
__device__ __forceinline__ float2* tap_ptr(float2* A, int base_phys, int L, int g, int k)
{
   if constexpr(LD::additive) return A + base_phys + LD::cphys(k * PL::stride(P));
   else                       return A + LD::phys(tap_pos<PL, P>(L, g, k));
}

template<class PL, int P, class LD>
__device__ __forceinline__ void lds_gather(float2 (&r)[PL::V], float2* A, int L)
{
   constexpr int R = PL::radix(P), G = PL::V / R;
#pragma unroll
   for(int g = 0; g < G; g++) {
      const int bp = LD::additive ? LD::phys(tap_pos<PL, P>(L, g, 0)) : 0;
#pragma unroll
      for(int k = 0; k < R; k++) r[g + k * G] = *tap_ptr<PL, P, LD>(A, bp, L, g, k);
   }
}

template<class PL, int P, class LD>
__device__ __forceinline__ void lds_scatter(const float2 (&r)[PL::V], float2* A, int L)
{
   constexpr int R = PL::radix(P), G = PL::V / R;
#pragma unroll
   for(int g = 0; g < G; g++) {
      const int bp = LD::additive ? LD::phys(tap_pos<PL, P>(L, g, 0)) : 0;
#pragma unroll
      for(int k = 0; k < R; k++) *tap_ptr<PL, P, LD>(A, bp, L, g, k) = r[g + k * G];
   }
}

// ---- stage twiddles --------------------------------------------------------------
// Every group keeps one base twiddle W^j and generates the rest by the
// reference's recurrences: the even/odd chains for radix 16, the single chain
// for radix 2/4/8 (fufft.cuh:436-450, 701-720, 743-746).  (Reading all stage
// twiddles from a table instead costs more: each lane's row lands in its own
// cache line, and the vector-memory path, not the VALU, becomes the limit.)
// Base twiddles depend only on the lane, so all of them are read once at
// kernel start: (cos, sin)(2*pi*j/P) serves the forward pass as (c, -s) and
// the inverse pass as (c, s).  Slot numbering: passes with M > 1 in order,
// G_p slots each.
template<class PL>
struct Twiddles {
   static constexpr int slots_before(int p)
   {
      int n = 0;
      for(int i = 0; i < p; i++)
         if(PL::stride(i) > 1) n += PL::V / PL::radix(i);
      return n;
   }
   static constexpr int COUNT = slots_before(PL::NP) > 0 ? slots_before(PL::NP) : 1;
   float2 w[COUNT];

   // the base twiddles of pass p, W^j of each of the lane's groups
   template<int p>
   __device__ __forceinline__ void load_pass(const Buf& tb, int L)
   {
      constexpr int R = PL::radix(p), M = PL::stride(p), G = PL::V / R;
      if constexpr(M > 1) {
#pragma unroll
         for(int g = 0; g < G; g++)
            w[slots_before(p) + g] = tb.ld2((uint32_t)(((L + g * PL::T) & (M - 1)) * 8), R * M * 8);
      }
   }

   __device__ __forceinline__ void load(const float2* table, int L)
   {
      const Buf tb(table, FUFFT_TW_ENTRIES * 8u);
      static_for<PL::NP>([&](auto pi) { load_pass<decltype(pi)::value>(tb, L); });
   }
};

// Stage twiddles carried from the forward DIF to the inverse DIT.  The
// forward's last twiddled pass (NP - 2: the last pass runs at M = 1) and the
// inverse's first twiddled pass are the same pass -- same lanes, same groups,
// same W^j -- and only the mid operation and the M = 1 butterflies lie between
// them, so the chain the forward pass generated is kept in registers and the
// inverse pass reads its conjugates instead of rebuilding it (R - 2 complex
// products per group).  Done where that pass has one group per lane (its
// radix is the lane radix) and the registers allow it:
//  - radix 8 (7 powers) at pure powers of 8 stays within 64 VGPRs, i.e. 8
//    wavefronts per SIMD; with a leading radix-2/4 pass (N = 1024, 2048, 8192)
//    the kept chain pushed it to 66-74 VGPRs, 6-7 wavefronts, which costs more
//    than it saves;
//  - radix 16 (15 powers) runs 4 wavefronts per SIMD, held by LDS, so up to
//    128 VGPRs are free: N = 256 and 4096 go from 77 to 110 VGPRs, N = 512 to
//    2048 (behind a lead pass) to 113-124; N = 8192 and 16384 would pass 128.
//    Same box: fp32 N = 4096 +1.1%, 1024 / 2048 +0.3 to +1%; BFP N = 4096
//    +1.5%, 1024 +2.9%, 2048 +1.3%.
// Results are unchanged bit for bit (tw_kept_conj).
template<class PL>
struct KeptChain {
   static constexpr int P = PL::NP >= 2 ? PL::NP - 2 : 0;
   static constexpr int R = PL::radix(P);
   static constexpr bool regs = PL::LEAD == 1 || (PL::V == 16 && PL::T <= 128);
   static constexpr bool enabled = PL::NP >= 2 && regs && R == PL::V && PL::stride(P) > 1;
   float2 w[enabled ? R : 1];
};

// KEEP: 0 plain; 1 forward pass that stores its chain in kc; 2 inverse pass
// that applies conj(kc)
enum { KEEP_NONE = 0, KEEP_STORE = 1, KEEP_USE = 2 };

// Butterflies + stage twiddles of pass P for all groups of the lane.
template<class PL, int P, int SIGN, bool DIT, int KEEP = KEEP_NONE>
__device__ __forceinline__ void compute_pass(float2 (&r)[PL::V], const Twiddles<PL>& tw, KeptChain<PL>& kc)
{
   constexpr int R = PL::radix(P), M = PL::stride(P), G = PL::V / R;
   constexpr bool keep = KeptChain<PL>::enabled && P == KeptChain<PL>::P && KEEP != KEEP_NONE;
   static_for<G>([&](auto gi) {
      constexpr int g = decltype(gi)::value;
      if constexpr(M > 1) {
         const float2 b = tw.w[Twiddles<PL>::slots_before(P) + g];
         const float2 w1 = SIGN < 0 ? make_float2(b.x, -b.y) : b;
         if constexpr(DIT) {
            if constexpr(keep && KEEP == KEEP_USE) tw_kept_conj<R, g, G>(r, kc.w);
            else                                   twiddle_group<R, CHAIN_EVENODD, g, G>(r, w1);
         }
         dftR<R, SIGN, g, G>(r);
         if constexpr(!DIT) {
            if constexpr(keep && KEEP == KEEP_STORE) {
               if constexpr(R == 16) chain_parity<g, G, true>(r, w1, kc.w);
               else                  chain_one<R, g, G>(r, w1, kc.w);
            }
            else                                     twiddle_group<R, CHAIN_EVENODD, g, G>(r, w1);
         }
      } else {
         dftR<R, SIGN, g, G>(r);
      }
   });
}

// Synchronisation of the exchange between pass P and pass P + 1.  WL is the
// number of consecutive lanes of one transform inside a wavefront (64, or T
// when a wavefront holds whole transforms, or 64/C for the column kernels).
// With one group per lane, pass P's lane L owns the positions
// (L / M) * R * M + (L % M) + k * M; when M <= WL the lane bits that pick the
// wavefront only reach the (L / M) part, so every wavefront owns one
// contiguous region of R * WL positions in pass P and in pass P + 1 alike and
// the exchange never leaves the wavefront: a wavefront fence suffices, and
// only exchanges across wavefronts need the workgroup barrier.  (Within a
// pass a lane writes back exactly the positions it read, so gather -> scatter
// of one pass needs no synchronisation at all.)
template<class PL, int P, int WL>
constexpr bool exchange_in_wave()
{
   if constexpr(PL::T <= WL) return true;
   else return PL::stride(P) <= WL && PL::V / PL::radix(P) == 1 && PL::V / PL::radix(P + 1) == 1;
}

template<class PL, int P, int LANES, int WL>
__device__ __forceinline__ void exchange_sync()
{
   if constexpr(exchange_in_wave<PL, P, WL>()) pass_barrier<64>();
   else                                        pass_barrier<LANES>();
}

// Forward DIF of the lane's registers: r holds positions L + q*T on entry and
// the digit-order spectrum positions L*V + k on exit (last pass at M = 1).
// With kc, the last twiddled pass leaves its chain there for inverse_dit.
template<class PL, class LD, int LANES, int WL = 64, int KEEP = KEEP_NONE>
__device__ __forceinline__ void forward_dif(float2 (&r)[PL::V], float2* A, int L, const Twiddles<PL>& tw,
                                            KeptChain<PL>& kc)
{
   static_for<PL::NP>([&](auto pi) {
      constexpr int p = decltype(pi)::value;
      if constexpr(p > 0) {
         exchange_sync<PL, p - 1, LANES, WL>();
         lds_gather<PL, p, typename LD::template at<PL, p - 1>>(r, A, L);
      }
      compute_pass<PL, p, -1, false, KEEP>(r, tw, kc);
      if constexpr(p < PL::NP - 1) lds_scatter<PL, p, typename LD::template at<PL, p>>(r, A, L);
   });
}

template<class PL, class LD, int LANES, int WL = 64>
__device__ __forceinline__ void forward_dif(float2 (&r)[PL::V], float2* A, int L, const Twiddles<PL>& tw)
{
   KeptChain<PL> none;
   forward_dif<PL, LD, LANES, WL, KEEP_NONE>(r, A, L, tw, none);
}

// Inverse DIT: r holds spectrum positions L*V + k on entry and natural-order
// positions L + q*T on exit.  With kc, the first twiddled pass applies the
// chain forward_dif kept.
template<class PL, class LD, int LANES, int WL = 64, int KEEP = KEEP_NONE>
__device__ __forceinline__ void inverse_dit(float2 (&r)[PL::V], float2* A, int L, const Twiddles<PL>& tw,
                                            KeptChain<PL>& kc)
{
   static_for<PL::NP>([&](auto qi) {
      constexpr int p = PL::NP - 1 - decltype(qi)::value;
      if constexpr(p < PL::NP - 1) lds_gather<PL, p, typename LD::template at<PL, p>>(r, A, L);
      compute_pass<PL, p, +1, true, KEEP>(r, tw, kc);
      if constexpr(p > 0) {
         lds_scatter<PL, p, typename LD::template at<PL, p - 1>>(r, A, L);
         exchange_sync<PL, p - 1, LANES, WL>();
      }
   });
}

template<class PL, class LD, int LANES, int WL = 64>
__device__ __forceinline__ void inverse_dit(float2 (&r)[PL::V], float2* A, int L, const Twiddles<PL>& tw)
{
   KeptChain<PL> none;
   inverse_dit<PL, LD, LANES, WL, KEEP_NONE>(r, A, L, tw, none);
}

// ---- digit order <-> natural order through LDS ------------------------------------------
// After the forward DIF lane L holds slots L*V + k, and slot L*V + k holds bin
// lane_bin(L) + k*T: digit p of the slot (weight M_p, radix R_p) becomes digit
// p of the bin (weight R_0 ... R_{p-1}); the last pass's digit is k itself.
template<class PL>
constexpr int digit_weight(int p)
{
   int w = 1;
   for(int i = 0; i < p; i++) w *= PL::radix(i);
   return w;
}

template<class PL>
__device__ __forceinline__ int lane_bin(int L)
{
   int f = 0;
   static_for<PL::NP - 1>([&](auto pi) {
      constexpr int p = decltype(pi)::value;
      constexpr int D = PL::stride(p) / PL::V;      // weight of digit p in the lane index
      f += ((L / D) & (PL::radix(p) - 1)) * digit_weight<PL>(p);
   });
   return f;
}

// Layout of the digit <-> natural exchange.  Its paired LDS accesses conflict
// when lanes of a quarter-wavefront (16 lanes, lane bits 0-3) hit slots that
// agree modulo 16.  The natural side touches L + q*T: those 16 lanes differ in
// bits 0-3.  The digit side touches lane_bin(L) + k*T: they differ in the bin
// bits where lane bits 0-3 land, most of them high.  phys = i ^ (each such
// high bin bit copied onto one of the bits 0-3 the bin does not already
// vary), so both sides cover 16 residues.  Bits from log2(T) up pass through,
// so offsets k*T and q*T stay additive (cphys(off) = off); the map is a
// bijection on [0, N) because bits 0-3 only receive bits above them.
template<class PL>
struct UnscrambleLds {
   // bit of lane_bin(L) that lane bit b becomes
   static constexpr int bin_bit(int b)
   {
      int w = 0;
      for(int p = 0; p < PL::NP - 1; p++) {
         const int d = ilog2c(PL::stride(p) / PL::V), r = ilog2c(PL::radix(p));
         if(b >= d && b < d + r) return w + b - d;
         w += r;
      }
      return -1;
   }
   struct Moves { int n = 0; int src[4] = {}; int dst[4] = {}; };
   static constexpr Moves moves()
   {
      Moves m;
      bool low[4] = {};
      for(int b = 0; b < 4; b++)
         if(bin_bit(b) >= 0 && bin_bit(b) < 4) low[bin_bit(b)] = true;
      int next = 0;
      for(int b = 0; b < 4; b++) {
         const int s = bin_bit(b);
         if(s < 4) continue;
         while(low[next]) next++;
         m.src[m.n] = s;
         m.dst[m.n] = next++;
         m.n++;
      }
      return m;
   }
   static constexpr Moves MV = moves();
   static constexpr bool additive = true;
   static_assert(PL::T >= 16, "a quarter-wavefront within one transform");

   __device__ __forceinline__ static int phys(int i)
   {
      int x = 0;
#pragma unroll
      for(int j = 0; j < MV.n; j++) x |= ((i >> MV.src[j]) & 1) << MV.dst[j];
      return i ^ x;
   }
   static constexpr int cphys(int off) { return off; }     // off is a multiple of T
};

// LDS slot of logical position base + off, where off is a multiple of V (so
// the padded layout stays additive)
template<class LD>
__device__ __forceinline__ float2* lds_slot(float2* A, int base_phys, int base, int off)
{
   if constexpr(LD::additive) return A + base_phys + LD::cphys(off);
   else                       return A + LD::phys(base + off);
}

// r[k] = slot L*V + k (forward DIF output)  ->  r[q] = bin L + q*T, so the
// store that follows is the coalesced natural-order store of the conv kernels.
// The first barrier orders the last DIF pass's gather before these writes.
// The exchange has its own layout (UnscrambleLds); the XOR layout, chosen at
// run time for comparison, keeps its own map.
template<class PL, class LD, int LANES>
__device__ __forceinline__ void digit_to_natural(float2 (&r)[PL::V], float2* A, int L)
{
   using UL = std::conditional_t<LD::additive, UnscrambleLds<PL>, LD>;
   constexpr int V = PL::V, T = PL::T;
   const int f = lane_bin<PL>(L);
   const int fp = UL::phys(f), lp = UL::phys(L);
   pass_barrier<LANES>();
#pragma unroll
   for(int k = 0; k < V; k++) *lds_slot<UL>(A, fp, f, k * T) = r[k];
   pass_barrier<LANES>();
#pragma unroll
   for(int q = 0; q < V; q++) r[q] = *lds_slot<UL>(A, lp, L, q * T);
}

// r[q] = bin L + q*T (natural-order load)  ->  r[k] = slot L*V + k, what the
// inverse DIT expects.  With WAR the trailing barrier orders these reads
// before the next pass's LDS writes.
template<class PL, class LD, int LANES, bool WAR>
__device__ __forceinline__ void natural_to_digit(float2 (&r)[PL::V], float2* A, int L)
{
   using UL = std::conditional_t<LD::additive, UnscrambleLds<PL>, LD>;
   constexpr int V = PL::V, T = PL::T;
   const int f = lane_bin<PL>(L);
   const int fp = UL::phys(f), lp = UL::phys(L);
#pragma unroll
   for(int q = 0; q < V; q++) *lds_slot<UL>(A, lp, L, q * T) = r[q];
   pass_barrier<LANES>();
#pragma unroll
   for(int k = 0; k < V; k++) r[k] = *lds_slot<UL>(A, fp, f, k * T);
   if constexpr(WAR) pass_barrier<LANES>();
}

// ---- the mid operation at the M = 1 boundary -----------------------------------------
// What a fused kernel does to each spectrum value between its forward and its
// inverse transform, in registers: the counterpart of the reference's Mid
// policies MidNothing / MidMultiply / MidConjMultiply (fufft.cuh:616-650),
// which rewrite the shared-memory buffer in a pass of their own.  As there, a
// new fusion costs a struct:
//
//    struct MidFoo {
//       static constexpr bool reads_filter = ...;   // false: no filter operand is read
//       __device__ static float2 apply(float2 a, float2 b);
//    };
//
// with a the spectrum value and b the filter value of the same slot (zero when
// reads_filter is false), plus one line in FUFFT_MID_POLICIES giving its id,
// the value the C ABI's `mid` argument takes.  Every kernel with a mid
// operation (the fused 1D and int16-BFP convs, the split apply, the 2D column
// kernels, the four-step middle) is then instantiated for it, and every entry
// point that takes `mid` accepts the id.
struct MidMultiply {
   static constexpr bool reads_filter = true;
   __device__ __forceinline__ static float2 apply(float2 a, float2 b) { return cmul(a, b); }
};
struct MidConjMultiply {
   static constexpr bool reads_filter = true;
   __device__ __forceinline__ static float2 apply(float2 a, float2 b) { return cmul_conj(a, b); }
};
struct MidNothing {
   static constexpr bool reads_filter = false;
   __device__ __forceinline__ static float2 apply(float2 a, float2) { return a; }
};

#define FUFFT_MID_POLICIES(X) \
   X(0, MidMultiply)          \
   X(1, MidConjMultiply)      \
   X(2, MidNothing)

// the ids of the three above, for the kernel kinds that fix their operation
enum { MID_MUL = 0, MID_CONJ = 1, MID_NONE = 2 };

template<int MID> struct MidById;
#define FUFFT_MID_BY_ID(id, S) template<> struct MidById<id> { using type = S; };
FUFFT_MID_POLICIES(FUFFT_MID_BY_ID)
#undef FUFFT_MID_BY_ID
template<int MID> using MidOf = typename MidById<MID>::type;
template<int MID> constexpr bool mid_reads_filter = MidOf<MID>::reads_filter;

// host side: is `mid` a registered id, and does its operation read a filter
constexpr bool mid_known(int mid)
{
#define FUFFT_MID_KNOWN(id, S) if(mid == id) return true;
   FUFFT_MID_POLICIES(FUFFT_MID_KNOWN)
#undef FUFFT_MID_KNOWN
   return false;
}
constexpr bool mid_needs_filter(int mid)
{
#define FUFFT_MID_FILTER(id, S) if(mid == id) return S::reads_filter;
   FUFFT_MID_POLICIES(FUFFT_MID_FILTER)
#undef FUFFT_MID_FILTER
   return false;
}

// f(std::integral_constant<int, id>{}) for the policy registered as `mid`;
// hipErrorInvalidValue for an unknown id
template<class F>
hipError_t with_mid(int mid, F&& f)
{
   switch(mid) {
#define FUFFT_MID_CASE(id, S) case id: return f(std::integral_constant<int, id>{});
      FUFFT_MID_POLICIES(FUFFT_MID_CASE)
#undef FUFFT_MID_CASE
      default: return hipErrorInvalidValue;
   }
}
// filter layouts: DR = digit order, slot i holds bin mixedrev(i) (what the
// reference's MidMultiply reads, fufft.cuh:635); LANE = the same values laid
// out lane-major in pairs, lane L's values 2m and 2m + 1 at 2(L + m*T) and
// 2(L + m*T) + 1 (lane_position; the reference's bperm, fufft.cuh:1444-1446,
// lays them out lane-major one value at a time), so that every 16-byte filter
// load of a wavefront reads one contiguous KiB; BPERM = the reference's bperm
// itself, lane L's k-th value at L + k*T (8-byte loads, one contiguous 512
// bytes per wavefront load), accepted so that its filters pass as they are
enum { FLT_DR = 0, FLT_LANE = 1, FLT_BPERM = 2 };

// The lane's V filter values as V/2 pairs, values 2m and 2m + 1 in the 16
// bytes at voff + m*mstep: mstep = 16 in digit order (the V values are
// contiguous), 16*T lane-major.  MID is a template parameter: a runtime
// branch between two products makes the compiler keep both results live
// across the join.
template<class PL, int MID, int POL = POL_DEFAULT>
__device__ __forceinline__ void mid_op_pairs(float2 (&r)[PL::V], const Buf& f, uint32_t voff, uint32_t mstep)
{
   using Op = MidOf<MID>;
   if constexpr(Op::reads_filter) {
      float2 b[PL::V];
#pragma unroll
      for(int m = 0; m < PL::V / 2; m++) {
         const float4 q = f.ld4<POL>(voff, m * mstep);
         b[2 * m] = make_float2(q.x, q.y);
         b[2 * m + 1] = make_float2(q.z, q.w);
      }
#pragma unroll
      for(int k = 0; k < PL::V; k++) r[k] = Op::apply(r[k], b[k]);
   } else {
#pragma unroll
      for(int k = 0; k < PL::V; k++) r[k] = Op::apply(r[k], make_float2(0.f, 0.f));
   }
}

// The two halves of load_dr_staged, for a caller that issues the loads early
// (the per-signal kernel, K_CONV_PSF_DR): the wavefront's V*64 contiguous
// slots from fslot0 + its first slot, 1 KiB per 16-byte load (POL: cache
// policy) ...
template<class PL, int POL = POL_DEFAULT>
__device__ __forceinline__ void dr_runs_load(float4 (&q)[PL::V / 2], const Buf& f, uint32_t fslot0, int L)
{
   constexpr int V = PL::V;
   static_assert(PL::T >= 64, "whole wavefronts per transform");
   const int wl = L & 63, w0 = (L & ~63) * V;      // lane in the wavefront, the wavefront's first slot
#pragma unroll
   for(int m = 0; m < V / 2; m++) q[m] = f.ld4<POL>((fslot0 + (uint32_t)w0) * 8u + (uint32_t)wl * 16u, m * 1024);
}

// ... and the hand-off to the lanes that hold those slots, through the LDS
// positions they hold in the last pass (layout LDL), which no other wavefront
// touches until this one's inverse reuses them (a wavefront fence)
template<class PL, class LDL>
__device__ __forceinline__ void dr_runs_stage(float2 (&b)[PL::V], const float4 (&q)[PL::V / 2], float2* A, int L)
{
   constexpr int V = PL::V;
   const int wl = L & 63, w0 = (L & ~63) * V;
#pragma unroll
   for(int m = 0; m < V / 2; m++) {
      const int s = w0 + m * 128 + 2 * wl;
      A[LDL::phys(s)]     = make_float2(q[m].x, q[m].y);
      A[LDL::phys(s + 1)] = make_float2(q[m].z, q[m].w);
   }
   pass_barrier<64>();
#pragma unroll
   for(int k = 0; k < V; k++) b[k] = A[LDL::phys(L * V + k)];
}

// The lane's V digit-order filter values, slots L*V .. L*V + V - 1 from
// fslot0, passed through LDS.  Read in place they are V/2 16-byte loads 16*V
// bytes apart, so a wavefront instruction touches 64 (V = 16) cache lines.
// The wavefront's 64*V slots are contiguous: it loads them in 1 KiB runs and
// writes them to the LDS positions its own lanes hold in the last pass
// (position L*V + k under that pass's layout LDL), which no other wavefront
// touches until this one's inverse scatters to them, so a wavefront fence
// orders the hand-over.  Needs whole wavefronts per transform (T >= 64).
template<class PL, class LDL>
__device__ __forceinline__ void load_dr_staged(float2 (&b)[PL::V], const Buf& f, uint32_t fslot0, float2* A, int L)
{
   float4 q[PL::V / 2];
   dr_runs_load<PL>(q, f, fslot0, L);
   dr_runs_stage<PL, LDL>(b, q, A, L);
}

template<class PL, class LDL, int MID>
__device__ __forceinline__ void mid_op_dr_staged(float2 (&r)[PL::V], const Buf& f, uint32_t fslot0, float2* A, int L)
{
   using Op = MidOf<MID>;
   float2 b[PL::V];
   load_dr_staged<PL, LDL>(b, f, fslot0, A, L);
#pragma unroll
   for(int k = 0; k < PL::V; k++) r[k] = Op::apply(r[k], b[k]);
}

// The lane's V filter values one at a time, value k at voff + k*kstep (the
// reference's bperm layout: T values apart; the 2D column kernels: one image
// row apart), read with cache policy POL.
template<class PL, int MID, int POL = POL_DEFAULT>
__device__ __forceinline__ void mid_op(float2 (&r)[PL::V], const Buf& f, uint32_t voff, uint32_t kstep)
{
   using Op = MidOf<MID>;
   if constexpr(Op::reads_filter) {
      float2 b[PL::V];
#pragma unroll
      for(int k = 0; k < PL::V; k++) b[k] = f.ld2<POL>(voff, k * kstep);
#pragma unroll
      for(int k = 0; k < PL::V; k++) r[k] = Op::apply(r[k], b[k]);
   } else {
#pragma unroll
      for(int k = 0; k < PL::V; k++) r[k] = Op::apply(r[k], make_float2(0.f, 0.f));
   }
}

}  // namespace fufft
