// Internal interface between the C-ABI layer (capi.hip) and the kernel
// translation units.  Not installed; the public contract is include/fufft/fufft.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace fufft {

// Dynamic LDS above 64 KiB must be allowed per kernel (and per device) before
// a launch.  Done once per (kernel, device) -- mask holds one bit per device
// -- so repeated launches, including launches under stream capture, make no
// attribute call.
inline hipError_t ensure_dynamic_lds(const void* kernel, size_t bytes, std::atomic<uint64_t>& mask)
{
   if(bytes <= 65536) return hipSuccess;
   int dev = 0;
   const hipError_t g = hipGetDevice(&dev);
   if(g != hipSuccess) return g;
   const uint64_t bit = 1ull << (dev & 63);
   if(mask.load(std::memory_order_acquire) & bit) return hipSuccess;
   const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
   if(e == hipSuccess) mask.fetch_or(bit, std::memory_order_acq_rel);
   return e;
}

// Lane-major filter and spectrum layout (FUFFT_LAYOUT_LANE) of an n-point
// plan with V = 2^vlog values per lane and T = n / V = 2^tlog lanes: lane L's
// digit-order slots L*V + 2m and L*V + 2m + 1 sit side by side at positions
// 2(L + m*T) and 2(L + m*T) + 1.  Each 16-byte load of a wavefront then reads
// one contiguous KiB (8 cache lines), where digit order spreads it over 64 or
// 32 lines.  lane_slot maps a position to the slot it holds, lane_position a
// slot to its position.
__host__ __device__ constexpr uint32_t lane_slot(uint32_t pos, uint32_t tlog, uint32_t vlog)
{
   return (((pos >> 1) & ((1u << tlog) - 1u)) << vlog) | ((pos >> (tlog + 1)) << 1) | (pos & 1u);
}
__host__ __device__ constexpr uint32_t lane_position(uint32_t slot, uint32_t tlog, uint32_t vlog)
{
   return (((slot >> vlog) | (((slot & ((1u << vlog) - 1u)) >> 1) << tlog)) << 1) | (slot & 1u);
}

// ---- 1D fused pipeline (conv1d.hip) ------------------------------------------------
// K_FWD_R2 / K_APPLY_R2: the forward half reading two real arrays, the
// inverse half writing two real arrays (2D two-for-one rows).
// K_C2C_FWD / K_C2C_INV: natural order in and out (forward DIF + digit ->
// natural exchange; natural -> digit exchange + inverse DIT, unnormalised).
// K_PLAN_TAPS: forward DIF of filter taps, times scale, stored in the filter
// layout fl (digit order or lane-major).
// K_CONV_TIMED: K_CONV with the phase timer (a timestamp after the load, the
// forward DIF, the mid operation, the inverse DIT and the store).
// K_CONV_MID: K_CONV as the four-step middle (N = 512 .. 4096), whose
// chunks the next launch reads again: default cache policy, where K_CONV
// streams its signal and result past the caches (POL_NT).
// K_CONV_PSF: K_CONV for one lane-major filter per signal at radix 16,
// N = 4096: the filter loads go out with the signal loads (without the kept
// twiddle chain, for the registers they hold through the forward DIF).
// K_CONV_PSF_DR: the same for one digit-order filter per signal (the
// reference's own per-signal format): the loads of each wavefront's 1 KiB
// filter runs go out with the signal loads, the hand-off to the lanes goes
// through LDS at the mid operation.
enum { K_CONV = 0, K_CONV_R2 = 1, K_FWD = 2, K_APPLY = 3, K_FWD_R2 = 4, K_APPLY_R2 = 5,
       K_C2C_FWD = 6, K_C2C_INV = 7, K_PLAN_TAPS = 8, K_CONV_TIMED = 9, K_CONV_MID = 10,
       K_CONV_PSF = 11, K_CONV_PSF_DR = 12 };

// the plans K_CONV_PSF and K_CONV_PSF_DR are built for: radix 16 with whole
// wavefronts per transform and room for the filter's 32 VGPRs within 128
// (N = 8192 would pass them).  Same box, 2^27 points, one filter per signal,
// bit-identical, Gpt/s against K_CONV: lane-major N = 1024 247.1 -> 254.0,
// 2048 258.2 -> 263.3, 4096 234.0 -> 243.4; digit order N = 2048 260.8 ->
// 268.0, 4096 239.5 -> 247.2, but N = 1024 258.6 -> 252.4: there
// K_CONV reads the digit-order filter in place (no LDS hand-off at T = 64),
// which the staged early read does not beat.
constexpr bool conv_psf_plan(int n, int v) { return v == 16 && (n == 1024 || n == 2048 || n == 4096); }
constexpr bool conv_psf_dr_plan(int n, int v) { return v == 16 && (n == 2048 || n == 4096); }
// the plan K_CONV_PSF runs with a late filter read, streamed past the caches
// (NT) as each filter is read once: radix 8 at N = 512, whose 8 wavefronts
// per SIMD leave no registers for an early read (263.7 -> 268.7 Gpt/s, same
// box, bit-identical).  At radix 16 N = 8192 / 16384, where an early read
// would pass 128 VGPRs, the late NT read measured 235.8 -> 215.8 and 217.0 ->
// 213.3, so those sizes keep the plain kernel.
constexpr bool conv_psf_late_plan(int n, int v) { return v == 8 && n == 512; }

// phase timer record of one workgroup (K_CONV_TIMED), TIMER_STRIDE words:
// [0] HW_ID, [1] XCC_ID, [2] marks, [3] s_memrealtime ticks (100 MHz) from
// the first mark to the last, [4..5] start (s_memtime, lo / hi),
// [6..10] one word per phase: phase id << 24 | cycles since start (saturated
// at 2^24 - 1), phases 1 load, 2 forward, 3 mid, 4 inverse, 5 store
enum { TIMER_STRIDE = 12, TIMER_MARKS = 5 };

struct Conv1dParams {
   const void*   in0;      // complex input, or real x (K_CONV_R2)
   const void*   in1;      // real y (K_CONV_R2)
   const void*   spec;     // spectrum (K_APPLY), laid out as sl says
   const void*   filt;     // filter, digit order or lane-major
   void*         out0;     // complex output / spectrum (K_FWD) / real u
   void*         out1;     // real v (K_CONV_R2)
   const float2* tw;       // device twiddle table
   uint32_t      ntrans;   // transforms in the launch
   uint32_t      fcount;   // transform t uses filter (t % fcount)
   uint32_t      scount;   // transform t uses spectrum (t % scount)
   int32_t       mid;      // a registered mid policy id (FUFFT_MID_POLICIES)
   int32_t       fl;       // FLT_DR / FLT_LANE (filter read; K_PLAN_TAPS: layout written)
   int32_t       sl;       // FLT_DR / FLT_LANE: spectrum K_FWD writes, K_APPLY reads
   float         scale;    // K_PLAN_TAPS: factor applied to the spectrum
   uint32_t*     timing;   // K_CONV_TIMED: TIMER_STRIDE words per workgroup
   uint32_t      timing_groups;   // workgroups that write a record
};

bool       conv1d_supported(int n, int v);
hipError_t launch_conv1d(int kind, int n, int v, int layout, const Conv1dParams& p, hipStream_t s);

// ---- fused conv at N = 32768, 32 values per lane (wide.hip) --------------------------
// The radix-16 plan (LEAD 8, three radix-16 passes) with each lane running two
// radix-16 lanes' groups; fufft_conv_f32 only (mid, filter layout and stride
// as there), results bit for bit the radix-16 plan's.
constexpr int CONV_WIDE_N = 32768;
constexpr bool conv_wide_plan(int64_t n, int v) { return n == CONV_WIDE_N && v == 16; }
// N = 16384 on the same kernel (512 lanes, 68 KiB of LDS: two workgroups per
// CU, where the workgroup kernel's 128 KiB allow one) for a shared lane-major
// filter: 227.5 -> 233.8 Gpt/s (same box, 2^27 points, 10 alternating
// rounds, bit-identical; 229.5 with its lead twiddles held, spilled).  With
// the digit-order filter (each lane's 128 contiguous bytes read in place) it
// measured 223.6 -> 192.3, with one lane-major filter per signal 219.2 ->
// 196.8, so those keep the workgroup kernel.
constexpr bool conv_wide_shared_lane_plan(int64_t n, int v) { return n == 16384 && v == 16; }
hipError_t launch_conv_wide(const Conv1dParams& p, int n, hipStream_t s);

// ---- filter planning on the device (plan.hip) ----------------------------------------
struct GatherDigits {
   int32_t np;             // digit groups (passes)
   int32_t bits;           // sum of the widths = log2 of the dimension
   uint8_t w[32];          // bit width of each group, in pass order
};
struct GatherParams {
   const float2* in;       // natural-order spectra
   float2*       out;      // planned filters (must not alias in)
   uint64_t      total;    // points over all items
   int32_t       lane_v;   // lane-major columns: values per lane of the row plan; 0 = digit order
   int32_t       bperm;    // with lane_v: the reference's bperm (slot L*V + k at L + k*T), not pairs
   float         scale;
   GatherDigits  dh, dw;   // rows (dh.np = 0 in 1D) and row digits
};
hipError_t launch_gather(const GatherParams& p, hipStream_t s);

// ---- int16 block floating point (bfp.hip) ---------------------------------------------
struct BfpParams {
   const void*   qin;      // int16 pairs
   const int8_t* ein;      // one exponent per block of 2^log_block points
   const void*   filt;     // fp32 filter
   void*         qout;
   int8_t*       eout;
   const float2* tw;
   uint32_t      ntrans;
   uint32_t      fcount;
   int32_t       mid;
   int32_t       fl;
   int32_t       log_block;   // 6 .. log2(n)
};

bool       bfp_supported(int n, int v);
hipError_t launch_bfp(int n, int v, int layout, const BfpParams& p, hipStream_t s);

// the reference's own format: one fp32 scale per transform, an int16 filter
struct BfpScaledParams {
   const void*   qin;      // int16 pairs
   const float*  sin;      // one scale per transform
   const void*   qfilt;    // int16 pairs, laid out as fl says
   const float*  sfilt;    // one scale per filter
   void*         qout;
   float*        sout;     // one scale per transform
   const float2* tw;
   uint32_t      ntrans;
   uint32_t      fcount;   // transform t uses filter (t % fcount)
   int32_t       mid;
   int32_t       fl;       // FLT_DR / FLT_LANE / FLT_BPERM, slots as in the fp32 filter
};

bool       bfp_scaled_supported(int n, int v);
hipError_t launch_bfp_scaled(int n, int v, const BfpScaledParams& p, hipStream_t s);

// ---- four-step outer levels (large.hip) -------------------------------------------
// one radix-16 level (stride M) over a batch of n-point transforms, in place;
// dit = false: forward DIF level, dit = true: inverse DIT level
// both outer levels of a two-level plan (n = 16 * 16 * mid, n >= 2^17) in one
// pass through LDS; bit-identical to the two single-level launches
hipError_t launch_outer2_pass(float2* buf, int64_t n, int64_t batch, bool dit, const float2* tw,
                              hipStream_t s);
hipError_t launch_outer_pass(float2* buf, int64_t n, int64_t batch, int64_t M, bool dit,
                             const float2* tw, hipStream_t s);

// ---- HBM stream ceiling (stream.hip) -------------------------------------------------
// copy of bytes (a multiple of 16) with 16-byte buffer loads and stores;
// nontemporal adds the NT cache policy
hipError_t launch_stream(const void* in, void* out, uint64_t bytes, bool nontemporal, hipStream_t s);
// the same copy in a given shape: workgroups of lanes (64, 256, 1024) lanes,
// loads (1 .. 32, a power of two) loads of width (8 or 16) bytes per lane in
// flight, per consecutive tiles per workgroup or (groups > 0) a persistent
// grid of that many workgroups, cache policies pld / pst (SC0 = 1, NT = 2)
bool stream_shape_ok(int lanes, int width, int loads, int per, int groups, int pld, int pst);
hipError_t launch_stream_shape(const void* in, void* out, uint64_t bytes, int lanes, int width, int loads,
                               int per, int groups, int pld, int pst, hipStream_t s);

// ---- 2D column kernels (conv2d.hip) -------------------------------------------------
struct ColParams {
   const void*   in;       // h x w complex images, rows contiguous (COL_CONV, COL_FWD)
   const void*   spec;     // 2D digit-order spectra (COL_APPLY)
   void*         out;
   const void*   filt;     // 2D filter: entry (r, c) = bin (rev_h(r), rev_w(slot(c)))
   const float2* tw;
   uint32_t      nimg;     // images in the launch
   uint32_t      fcount;   // image i uses filter (i % fcount)
   uint32_t      scount;   // image i uses spectrum (i % scount)
   int32_t       mid;
   uint32_t      w;        // row length
   // Filter column order.  f_dr = 0: the filter's columns are in the row
   // spectra's lane-major order, so column c reads filter column c.  f_dr = 1:
   // the reference's order, entry (r, s) = bin (rev_h(r), rev_w(s)); column c
   // holds row slot s = lane_slot(c, f_tr_log, f_vr_log) (V = 2^f_vr_log values
   // per lane of the row plan, T = w / V = 2^f_tr_log) and reads filter column s.
   uint32_t      f_dr;
   uint32_t      f_tr_log;
   uint32_t      f_vr_log;
};
enum { COL_CONV = 0, COL_FWD = 1, COL_APPLY = 2 };
int        col_values_per_lane(int h);      // 0 if h is not a supported column length
hipError_t launch_col(int kind, int h, const ColParams& p, hipStream_t s);

// ---- small images: the whole 2D conv in one workgroup (conv2d.hip) --------------------
struct Small2dParams {
   const void*   in;       // h x w complex images, rows contiguous
   void*         out;
   const void*   filt;     // 2D filter, entry (r, c) = bin (rev_h(r), rev_w(c)), radix 8 both ways
   const float2* tw;
   uint32_t      nimg;
   uint32_t      fcount;   // image i uses filter (i % fcount)
   int32_t       mid;
};
bool       small2d_supported(int64_t h, int64_t w);
hipError_t launch_small2d(int h, int w, const Small2dParams& p, hipStream_t s);

}  // namespace fufft
