// fuFFT for MI355X -- header-only C++ mirror of the reference's launch surface.
//
// The reference is driven from C++ by instantiating kernel templates with a
// Mid policy type (MidMultiply / MidConjMultiply / MidNothing, fufft.cuh:
// 616-650) and launching them (bench_fufft.cu:216-221, 446-450).  This header
// keeps that shape -- the Mid policy is a template argument -- and forwards to
// the C ABI in fufft.h, so C++ callers port by swapping the launch for a call.
// Pointers are device pointers to interleaved complex float; every function
// returns the C ABI status (FUFFT_OK = 0).  Nothing here allocates.
#ifndef FUFFT_FUFFT_HPP
#define FUFFT_FUFFT_HPP

#include <cstddef>
#include <cstdint>
#include <type_traits>
#include <vector>

#include "fufft.h"

namespace fufft {

// Mid policies: the reference's functor types, reduced to the C ABI ids (the
// device side of each is a struct of the library's kernel sources).  As in
// the reference (fufft.cuh:625-650), MidMultiply{b} and MidConjMultiply{b}
// carry their filter, for the launch surface of namespace fufft::ref below;
// the functions above that namespace take the filter as an argument and use
// the types only as tags.
struct MidMultiply     { static constexpr int id = FUFFT_MID_MUL;  const void* b = nullptr; };
struct MidConjMultiply { static constexpr int id = FUFFT_MID_CONJ; const void* b = nullptr; };
struct MidNothing      { static constexpr int id = FUFFT_MID_NONE; };
// 1: the policy `mid` reads a filter; 0: it reads none; FUFFT_ERR_INVALID: no such policy
inline int mid_reads_filter(int mid) { return fufft_mid_reads_filter(mid); }
template<class Mid> inline bool reads_filter() { return fufft_mid_reads_filter(Mid::id) == 1; }

enum class Variant : int { V16 = FUFFT_V16, R8 = FUFFT_R8, Auto = FUFFT_AUTO };

inline const char* status_string(int status) { return fufft_status_string(status); }
// true when the loaded library was built from this header (FUFFT_ABI_VERSION)
inline bool abi_matches() { return fufft_abi_version() == FUFFT_ABI_VERSION; }
inline int init(int device = 0) { return fufft_init(device); }
inline bool supported(int64_t n, Variant v = Variant::Auto) { return fufft_supported(n, (int)v) != 0; }
// the faster variant for a filter layout (FUFFT_LAYOUT_LANE: radix 16 from n = 1024 on);
// returns FUFFT_OK, or the library's negative status (an unsupported n or an
// unknown layout) with *out left unchanged
inline int fastest_variant(int64_t n, Variant* out, int layout = FUFFT_LAYOUT_LANE)
{
   const int v = fufft_fastest_variant(n, layout);
   if(v < 0) return v;
   if(out) *out = v == FUFFT_R8 ? Variant::R8 : Variant::V16;
   return FUFFT_OK;
}

// ---- host planning (bench_fufft.cu:63-82, 156-170) ---------------------------------------

// natural-order spectrum (kind FUFFT_FILTER_SPECTRUM) or taps (FUFFT_FILTER_TAPS)
// -> the filter the kernels read, 1/n folded in
inline int plan_filter(const float* natural, float* planned, int64_t n, Variant v = Variant::Auto,
                       int kind = FUFFT_FILTER_TAPS, int layout = FUFFT_LAYOUT_DR, bool fold_inv_n = true)
{
   return fufft_plan_filter_f32(n, (int)v, layout, kind, fold_inv_n ? 1 : 0, natural, planned);
}

inline std::vector<int32_t> digit_order(int64_t n, Variant v = Variant::Auto)
{
   std::vector<int32_t> perm(static_cast<std::size_t>(n));
   if(fufft_digit_order(n, (int)v, perm.data()) != FUFFT_OK) perm.clear();
   return perm;
}

// ---- 1D fused path ------------------------------------------------------------------------

// fufft_pipeline_v16 / _ip / _fused<..., Mid> (fufft.cuh:1499-1534, 1757-1791)
template<class Mid = MidMultiply>
inline int pipeline(const void* in, const void* filt, void* out, int64_t n, int64_t batch,
                    void* stream = nullptr, int64_t filt_stride = 0, Variant v = Variant::Auto,
                    int layout = FUFFT_LAYOUT_DR)
{
   return fufft_conv_f32(in, filt, filt_stride, out, n, batch, Mid::id, (int)v, layout, stream);
}

// fufft_pipeline_fwd (fufft.cuh:1343-1370)
inline int pipeline_fwd(const void* in, void* spec, int64_t n, int64_t batch, void* stream = nullptr,
                        Variant v = Variant::Auto)
{
   return fufft_fwd_f32(in, spec, n, batch, (int)v, stream);
}

// fufft_pipeline_apply<Mid> (fufft.cuh:1372-1407); spec_stride 0 broadcasts one spectrum
template<class Mid = MidMultiply>
inline int pipeline_apply(const void* spec, const void* filt, void* out, int64_t n, int64_t batch,
                          void* stream = nullptr, int64_t spec_stride = 0, int64_t filt_stride = 0,
                          Variant v = Variant::Auto, int layout = FUFFT_LAYOUT_DR)
{
   return fufft_apply_f32(spec, spec_stride, filt, filt_stride, out, n, batch, Mid::id, (int)v, layout,
                          stream);
}

// fufft_conv_r2 (fufft.cuh:1273-1330): two real signals, real filter
inline int conv_r2(const float* x, const float* y, const void* filt, float* u, float* v, int64_t n,
                   int64_t batch, void* stream = nullptr, int64_t filt_stride = 0,
                   Variant var = Variant::Auto, int layout = FUFFT_LAYOUT_DR)
{
   return fufft_conv_r2_f32(x, y, filt, filt_stride, u, v, n, batch, (int)var, layout, stream);
}

// fufft_pipeline_v16_bfp<Mid> (fufft.cuh:1614-1701), int8 exponent per block of
// `block` points (64 by default; block = n: one exponent per transform)
template<class Mid = MidMultiply>
inline int pipeline_bfp(const void* qin, const int8_t* ein, const void* filt, void* qout, int8_t* eout,
                        int64_t n, int64_t batch, void* stream = nullptr, int64_t filt_stride = 0,
                        Variant v = Variant::Auto, int layout = FUFFT_LAYOUT_DR,
                        int64_t block = FUFFT_BFP_BLOCK)
{
   return fufft_conv_bfp16(qin, ein, filt, filt_stride, qout, eout, n, batch, block, Mid::id, (int)v,
                           layout, stream);
}

// fufft_pipeline_v16_bfp<Mid>(aq, a_scale, bq, b_scale, outq, out_scale) (fufft.cuh:1614-1701)
// in its own format: one fp32 scale per transform, an int16 filter (the reference's digit
// order by default) with one scale per filter (filt_stride 0: one filter; n: one per transform)
template<class Mid = MidMultiply>
inline int pipeline_bfp_scaled(const void* aq, const float* a_scale, const void* bq, const float* b_scale,
                               void* outq, float* out_scale, int64_t n, int64_t batch,
                               void* stream = nullptr, int64_t filt_stride = 0, Variant v = Variant::V16,
                               int layout = FUFFT_LAYOUT_DR)
{
   return fufft_conv_bfp16_scaled(aq, a_scale, bq, b_scale, filt_stride, outq, out_scale, n, batch, Mid::id,
                                  (int)v, layout, stream);
}

// fufft_c2c<N, LOG8N, CPB> (fufft.cuh:879-904): natural-order batched C2C; the
// reference's is forward only, Direction here is FUFFT_FORWARD or FUFFT_INVERSE
template<int Direction = FUFFT_FORWARD>
inline int c2c(const void* in, void* out, int64_t n, int64_t batch, void* stream = nullptr,
               Variant v = Variant::Auto)
{
   static_assert(Direction == FUFFT_FORWARD || Direction == FUFFT_INVERSE, "direction is -1 or +1");
   return fufft_c2c_f32(in, out, n, batch, Direction, (int)v, stream);
}

// the host planning of bench_fufft.cu:156-170 on device memory, for count filters
inline int plan_filter_device(const void* natural, void* planned, int64_t n, int64_t count = 1,
                              void* stream = nullptr, Variant v = Variant::Auto,
                              int kind = FUFFT_FILTER_TAPS, int layout = FUFFT_LAYOUT_DR,
                              bool fold_inv_n = true)
{
   return fufft_plan_filter_device_f32(natural, planned, n, count, (int)v, layout, kind,
                                       fold_inv_n ? 1 : 0, stream);
}

// the reference's FUFFT_TIMER_* in-kernel phase marks (fufft.cuh:86-176) around a fused conv:
// timing receives FUFFT_TIMER_STRIDE words per workgroup for the first timing_groups workgroups
template<class Mid = MidMultiply>
inline int pipeline_timed(const void* in, const void* filt, void* out, int64_t n, int64_t batch,
                          uint32_t* timing, int64_t timing_groups, void* stream = nullptr,
                          int64_t filt_stride = 0, Variant v = Variant::Auto, int layout = FUFFT_LAYOUT_DR)
{
   return fufft_conv_timed_f32(in, filt, filt_stride, out, n, batch, Mid::id, (int)v, layout, timing,
                               timing_groups, stream);
}

// the four-step chain order of the reference's V=16 middle by default (bench_fufft.cu:410-428)
inline int plan_filter_large_device(const void* natural, void* planned, int64_t n, int64_t count = 1,
                                    void* stream = nullptr, int kind = FUFFT_FILTER_TAPS, bool fold_inv_n = true,
                                    Variant middle = Variant::V16)
{
   return fufft_plan_filter_large_device_f32(natural, planned, n, count, (int)middle, kind, fold_inv_n ? 1 : 0,
                                             stream);
}

// 2D filters default to the reference's column order (verify_kernel.cpp:738-748);
// FUFFT_LAYOUT_LANE is this library's faster order (fufft.h, 2D section)
inline int plan_filter2d_device(const void* natural, void* planned, int64_t h, int64_t w, int64_t count = 1,
                                void* stream = nullptr, int kind = FUFFT_FILTER_TAPS, bool fold_inv_n = true,
                                int layout = FUFFT_LAYOUT_DR)
{
   return fufft_plan_filter2d_device_f32(natural, planned, h, w, count, layout, kind, fold_inv_n ? 1 : 0,
                                         stream);
}

// ---- four-step (run_large, bench_fufft.cu:357-492) ----------------------------------------

// run_large<N, LOUT, 16, MID, lead, nrv>: the middle is fufft_pipeline_v16 (Variant::V16)
template<class Mid = MidMultiply>
inline int conv_large(void* buf, const void* filt, int64_t n, int64_t batch, void* stream = nullptr,
                      int64_t filt_stride = 0, Variant middle = Variant::V16)
{
   return fufft_conv_large_f32(buf, filt, filt_stride, n, batch, Mid::id, (int)middle, stream);
}

// ---- 2D (fufft_conv2d, fufft.cuh:1209-1258) -------------------------------------------------

template<class Mid = MidMultiply>
inline int conv2d(const void* in, const void* filt, void* out, int64_t h, int64_t w, int64_t batch,
                  void* stream = nullptr, int64_t filt_stride = 0, int layout = FUFFT_LAYOUT_DR)
{
   return fufft_conv2d_f32(in, filt, filt_stride, out, h, w, batch, Mid::id, layout, stream);
}

inline int conv2d_r2(const float* x, const float* y, const void* filt, float* u, float* v, void* work,
                     int64_t h, int64_t w, int64_t batch, void* stream = nullptr, int64_t filt_stride = 0,
                     int layout = FUFFT_LAYOUT_DR)
{
   return fufft_conv2d_r2_f32(x, y, filt, filt_stride, u, v, work, h, w, batch, layout, stream);
}

inline int fwd2d(const void* in, void* spec, int64_t h, int64_t w, int64_t batch, void* stream = nullptr)
{
   return fufft_fwd2d_f32(in, spec, h, w, batch, stream);
}

template<class Mid = MidMultiply>
inline int apply2d(const void* spec, const void* filt, void* out, int64_t h, int64_t w, int64_t batch,
                   void* stream = nullptr, int64_t spec_stride = 0, int64_t filt_stride = 0,
                   int layout = FUFFT_LAYOUT_DR)
{
   return fufft_apply2d_f32(spec, spec_stride, filt, filt_stride, out, h, w, batch, Mid::id, layout, stream);
}

// ---- the reference's launch surface, by name --------------------------------------------
// A caller of the reference instantiates a kernel template whose parameters
// spell out the plan and launches it, e.g. (bench_fufft.cu:216-221)
//
//    fufft_pipeline_v16<N, L16, NR16, CPB><<<batch / CPB, CPB * N / 16, CPB * N * 8>>>(
//       d_a, d_out, MidMultiply{d_b16}, nullptr);
//
// The functions of fufft::ref keep those names, template parameters and
// pointer arguments, so that launch becomes
//
//    fufft::ref::fufft_pipeline_v16<N, L16, NR16, CPB>(d_a, d_out, MidMultiply{d_b16}, batch, stream);
//
// - The template parameters are checked at compile time against the plan the
//   library runs for them: N = LEAD * 16^NRV (LEAD 1, 2, 4 or 8) for the
//   radix-16 kernels, N = LEAD * 8^NR8 (LEAD 1, 2 or 4) for the radix-8 ones,
//   the reference's own plans (cpu_mixed.cpp:36-49), whose digit order the
//   filter is in.  A template the library cannot run as written is a compile
//   error, not a silently different plan.
// - CPB, the reference's transforms per block, is launch geometry: checked
//   as the reference checks it (>= 1; at most 16 for the BFP kernel,
//   fufft.cuh:1621) and otherwise unused, since the library chooses its own.
//   Any batch works (the reference needs a multiple of CPB).
// - Filters are per transform, as every one of these kernels reads them
//   (b[base + i], fufft.cuh:635; bperm[base + ...], 1476; b_scale[tix],
//   1638): filter t of the batch at b + t*N, in the plan's digit order
//   (bperm for the _v16f / _fused kernels).
// - The results are the library's, bit for bit the oracle's restatement of
//   the same kernel; with fufft_set_twiddles(FUFFT_TWIDDLES_REFERENCE) they are
//   the reference's own CPU transcription's.
// - The return value is the C ABI status (FUFFT_OK = 0): the launch is
//   asynchronous on `stream`, and nothing allocates.
namespace ref {

using fufft::MidConjMultiply;
using fufft::MidMultiply;
using fufft::MidNothing;

namespace plan {
constexpr int64_t ipow(int64_t b, int e) { return e <= 0 ? 1 : b * ipow(b, e - 1); }
// the radix-16 plans: LEAD then NRV radix-16 passes
constexpr bool v16(int64_t n, int lead, int nrv)
{
   return (lead == 1 || lead == 2 || lead == 4 || lead == 8) && nrv >= 1 && n == lead * ipow(16, nrv);
}
// the radix-8 plans: LEAD then NR8 radix-8 passes
constexpr bool r8(int64_t n, int lead, int nr8)
{
   return (lead == 1 || lead == 2 || lead == 4) && nr8 >= 1 && n == lead * ipow(8, nr8);
}
template<class Mid> constexpr bool is_mid()
{
   return std::is_same<Mid, MidMultiply>::value || std::is_same<Mid, MidConjMultiply>::value ||
          std::is_same<Mid, MidNothing>::value;
}
// the filter a Mid carries (none for MidNothing) and its stride: one per transform
template<class Mid> inline const void* filter_of(const Mid& m) { return m.b; }
inline const void* filter_of(const MidNothing&) { return nullptr; }
template<class Mid> constexpr int64_t stride_of(int64_t n) { return std::is_same<Mid, MidNothing>::value ? 0 : n; }
}  // namespace plan

// fufft_pipeline_v16<N, LEAD, NRV, CPB> (fufft.cuh:1518-1534): the radix-16
// fused conv.  The reference's takes MidMultiply only; any Mid works here.
template<int N, int LEAD, int NRV, int CPB, class Mid = MidMultiply>
inline int fufft_pipeline_v16(const void* a, void* out, Mid mid, int64_t batch, void* stream = nullptr)
{
   static_assert(plan::v16(N, LEAD, NRV), "fufft_pipeline_v16: N must be LEAD * 16^NRV, LEAD in {1, 2, 4, 8}");
   static_assert(CPB >= 1, "fufft_pipeline_v16: CPB >= 1");
   static_assert(plan::is_mid<Mid>(), "Mid: MidMultiply, MidConjMultiply or MidNothing");
   return fufft_conv_f32(a, plan::filter_of(mid), plan::stride_of<Mid>(N), out, N, batch, Mid::id, FUFFT_V16,
                         FUFFT_LAYOUT_DR, stream);
}

// fufft_pipeline_v16_wide<N, LEAD, NRV, CPB> (fufft.cuh:1717-1734): the same
// conv for middles above 4096 in the reference; one entry here
template<int N, int LEAD, int NRV, int CPB, class Mid = MidMultiply>
inline int fufft_pipeline_v16_wide(const void* a, void* out, Mid mid, int64_t batch, void* stream = nullptr)
{
   return fufft_pipeline_v16<N, LEAD, NRV, CPB, Mid>(a, out, mid, batch, stream);
}

// fufft_pipeline_v16f<N, LEAD, NRV, CPB> (fufft.cuh:1499-1516): the filter in
// the reference's bperm layout (bperm[L + k*T] = b_dr[16L + k] per transform)
template<int N, int LEAD, int NRV, int CPB>
inline int fufft_pipeline_v16f(const void* a, const void* bperm, void* out, int64_t batch, void* stream = nullptr)
{
   static_assert(plan::v16(N, LEAD, NRV), "fufft_pipeline_v16f: N must be LEAD * 16^NRV, LEAD in {1, 2, 4, 8}");
   static_assert(CPB >= 1, "fufft_pipeline_v16f: CPB >= 1");
   return fufft_conv_f32(a, bperm, N, out, N, batch, FUFFT_MID_MUL, FUFFT_V16, FUFFT_LAYOUT_BPERM, stream);
}

// fufft_pipeline_ip<N, LEAD, NR8, CPB, Mid> (fufft.cuh:1757-1772): the radix-8 conv
template<int N, int LEAD, int NR8, int CPB, class Mid>
inline int fufft_pipeline_ip(const void* a, void* out, Mid mid, int64_t batch, void* stream = nullptr)
{
   static_assert(plan::r8(N, LEAD, NR8), "fufft_pipeline_ip: N must be LEAD * 8^NR8, LEAD in {1, 2, 4}");
   static_assert(CPB >= 1, "fufft_pipeline_ip: CPB >= 1");
   static_assert(plan::is_mid<Mid>(), "Mid: MidMultiply, MidConjMultiply or MidNothing");
   return fufft_conv_f32(a, plan::filter_of(mid), plan::stride_of<Mid>(N), out, N, batch, Mid::id, FUFFT_R8,
                         FUFFT_LAYOUT_DR, stream);
}

// fufft_pipeline_fused<N, LEAD, NR8, CPB> (fufft.cuh:1774-1791): radix 8, bperm filter
template<int N, int LEAD, int NR8, int CPB>
inline int fufft_pipeline_fused(const void* a, const void* bperm, void* out, int64_t batch, void* stream = nullptr)
{
   static_assert(plan::r8(N, LEAD, NR8), "fufft_pipeline_fused: N must be LEAD * 8^NR8, LEAD in {1, 2, 4}");
   static_assert(CPB >= 1, "fufft_pipeline_fused: CPB >= 1");
   return fufft_conv_f32(a, bperm, N, out, N, batch, FUFFT_MID_MUL, FUFFT_R8, FUFFT_LAYOUT_BPERM, stream);
}

// fufft_pipeline_v16_bfp<N, LEAD, NRV, CPB> (fufft.cuh:1614-1701): int16
// pairs with one fp32 scale per transform in and out, an int16 filter with
// one scale per transform (bq, b_scale), the reference's codec
// (fufft_bfp_scaled_quantize)
template<int N, int LEAD, int NRV, int CPB>
inline int fufft_pipeline_v16_bfp(const void* aq, const float* a_scale, const void* bq, const float* b_scale,
                                  void* outq, float* out_scale, int64_t batch, void* stream = nullptr)
{
   static_assert(plan::v16(N, LEAD, NRV), "fufft_pipeline_v16_bfp: N must be LEAD * 16^NRV, LEAD in {1, 2, 4, 8}");
   static_assert(CPB >= 1 && CPB <= 16, "fufft_pipeline_v16_bfp: 1 <= CPB <= 16 (fufft.cuh:1621)");
   return fufft_conv_bfp16_scaled(aq, a_scale, bq, b_scale, N, outq, out_scale, N, batch, FUFFT_MID_MUL,
                                  FUFFT_V16, FUFFT_LAYOUT_DR, stream);
}

// fufft_pipeline_fwd / fufft_pipeline_apply<N, LEAD, NR8, CPB> (fufft.cuh:
// 1343-1407): the split radix-8 path; apply reads spectrum and filter per
// transform (spec[base + i], bspec_dr[base + i])
template<int N, int LEAD, int NR8, int CPB>
inline int fufft_pipeline_fwd(const void* a, void* spec, int64_t batch, void* stream = nullptr)
{
   static_assert(plan::r8(N, LEAD, NR8), "fufft_pipeline_fwd: N must be LEAD * 8^NR8, LEAD in {1, 2, 4}");
   static_assert(CPB >= 1, "fufft_pipeline_fwd: CPB >= 1");
   return fufft_fwd_f32(a, spec, N, batch, FUFFT_R8, stream);
}

template<int N, int LEAD, int NR8, int CPB>
inline int fufft_pipeline_apply(const void* spec, const void* bspec_dr, void* out, int64_t batch,
                                void* stream = nullptr)
{
   static_assert(plan::r8(N, LEAD, NR8), "fufft_pipeline_apply: N must be LEAD * 8^NR8, LEAD in {1, 2, 4}");
   static_assert(CPB >= 1, "fufft_pipeline_apply: CPB >= 1");
   return fufft_apply_f32(spec, N, bspec_dr, N, out, N, batch, FUFFT_MID_MUL, FUFFT_R8, FUFFT_LAYOUT_DR, stream);
}

// fufft_conv_r2<N, LEAD, NR8, CPB> (fufft.cuh:1273-1330): two real signals per
// complex transform against a real filter's spectrum, per transform
template<int N, int LEAD, int NR8, int CPB>
inline int fufft_conv_r2(const float* xr, const float* yr, const void* bspec_dr, float* ur, float* vr,
                         int64_t batch, void* stream = nullptr)
{
   static_assert(plan::r8(N, LEAD, NR8), "fufft_conv_r2: N must be LEAD * 8^NR8, LEAD in {1, 2, 4}");
   static_assert(CPB >= 1, "fufft_conv_r2: CPB >= 1");
   return fufft_conv_r2_f32(xr, yr, bspec_dr, N, ur, vr, N, batch, FUFFT_R8, FUFFT_LAYOUT_DR, stream);
}

// fufft_conv2d<H, W, CPB> (fufft.cuh:1209-1258): the fused 2D conv, filter
// entry (r, c) = bin (rev_H(r), rev_W(c)) per image (verify_kernel.cpp:738-748)
template<int H, int W, int CPB>
inline int fufft_conv2d(const void* a, void* out, MidMultiply mid, int64_t batch, void* stream = nullptr)
{
   static_assert(H >= 8 && W >= 8 && (H & (H - 1)) == 0 && (W & (W - 1)) == 0,
                 "fufft_conv2d: H and W powers of two from 8");
   static_assert(CPB >= 1, "fufft_conv2d: CPB >= 1");
   return fufft_conv2d_f32(a, mid.b, (int64_t)H * W, out, H, W, batch, FUFFT_MID_MUL, FUFFT_LAYOUT_DR, stream);
}

// fufft_c2c<N, LOG8N, CPB> (fufft.cuh:878-904): the forward natural-order C2C
template<int N, int LOG8N, int CPB>
inline int fufft_c2c(const void* in, void* out, int64_t batch, void* stream = nullptr)
{
   static_assert(LOG8N >= 1 && N == plan::ipow(8, LOG8N), "fufft_c2c: N must be 8^LOG8N");
   static_assert(CPB >= 1, "fufft_c2c: CPB >= 1");
   return fufft_c2c_f32(in, out, N, batch, FUFFT_FORWARD, FUFFT_R8, stream);
}

// run_large<N, LOUT, ROUT, MID, MLEAD, MNRV> (bench_fufft.cu:399-450): the
// four-step chain in place, LOUT radix-16 outer levels around the
// fufft_pipeline_v16 middle of MID = MLEAD * 16^MNRV points, the filter in
// the chain order of bench_fufft.cu:410-428, one per transform.  The library
// splits each N one way (fufft_large_plan); a split it does not run returns
// FUFFT_ERR_UNSUPPORTED before any launch (its filter order would differ).
template<int N, int LOUT, int ROUT, int MID, int MLEAD, int MNRV>
inline int run_large(void* buf, const void* bdr, int64_t batch, void* stream = nullptr)
{
   static_assert(ROUT == 16, "run_large: the outer levels are radix 16");
   static_assert(LOUT >= 1 && plan::v16(MID, MLEAD, MNRV) && (int64_t)N == plan::ipow(16, LOUT) * MID,
                 "run_large: N must be 16^LOUT * MID and MID = MLEAD * 16^MNRV, MLEAD in {1, 2, 4, 8}");
   int lout = 0, mid = 0;
   if(fufft_large_plan(N, &lout, &mid) != FUFFT_OK || lout != LOUT || mid != MID) return FUFFT_ERR_UNSUPPORTED;
   return fufft_conv_large_f32(buf, bdr, N, N, batch, FUFFT_MID_MUL, FUFFT_V16, stream);
}

}  // namespace ref

}  // namespace fufft

#endif  // FUFFT_FUFFT_HPP
