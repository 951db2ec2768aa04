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
#include <vector>

#include "fufft.h"

namespace fufft {

// Mid policies: the reference's functor types, reduced to the C ABI ids (the
// device side of each is a struct of the library's kernel sources).
struct MidMultiply     { static constexpr int id = FUFFT_MID_MUL; };
struct MidConjMultiply { static constexpr int id = FUFFT_MID_CONJ; };
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

}  // namespace fufft

#endif  // FUFFT_FUFFT_HPP
