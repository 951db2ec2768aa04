// fuFFT for MI355X -- C++ plan objects over the C ABI.
//
// The reference's caller carries three facts by hand from filter planning to
// launch (bench_fufft.cu:156-221, 410-450): which kernel template it runs
// (fufft_pipeline_v16 or fufft_pipeline_ip, the four-step middle), the digit
// order that template implies (mixedrev_host over its radices, or the chain
// order), and the device buffer the permuted, 1/N-scaled filter was copied
// to.  The filter array itself cannot say which order it is in, so a filter
// launched with another plan gives wrong output without an error.
//
// A plan object here owns its device filter and remembers the plan it was
// made for: the variant (resolved at construction -- Variant::Auto becomes the
// fastest variant for the chosen layout), the filter layout and the filter
// count.  Every launch through the object passes that plan, so a filter and
// its launch cannot disagree.  The objects allocate in their constructors
// (hipMalloc, one buffer per plan) and never in a launch; launches are
// asynchronous on the given stream, exactly as the C calls they make.
// Errors throw fufft::Error carrying the C ABI status; arguments are checked
// before any allocation or device call.
//
// Requires the HIP runtime headers and library (hipMalloc / hipMemcpy /
// hipFree); include/fufft/fufft.hpp alone needs neither.
#ifndef FUFFT_PLAN_HPP
#define FUFFT_PLAN_HPP

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "fufft.hpp"

namespace fufft {

class Error : public std::runtime_error {
public:
   Error(int status, const std::string& where)
      : std::runtime_error(where + ": " + fufft_status_string(status)), status_(status) {}
   int status() const noexcept { return status_; }

private:
   int status_;
};

inline void check(int status, const char* where)
{
   if(status != FUFFT_OK) throw Error(status, where);
}

inline void check_hip(hipError_t e, const char* where)
{
   if(e != hipSuccess) throw Error(FUFFT_ERR_HIP, std::string(where) + " (" + hipGetErrorString(e) + ")");
}

// A device allocation owned by a plan: hipMalloc on construction, hipFree on
// destruction; movable, not copyable.
class DeviceBuffer {
public:
   DeviceBuffer() = default;
   explicit DeviceBuffer(std::size_t bytes) : bytes_(bytes)
   {
      if(bytes) check_hip(hipMalloc(&p_, bytes), "hipMalloc");
   }
   ~DeviceBuffer() { release(); }
   DeviceBuffer(const DeviceBuffer&) = delete;
   DeviceBuffer& operator=(const DeviceBuffer&) = delete;
   DeviceBuffer(DeviceBuffer&& o) noexcept : p_(std::exchange(o.p_, nullptr)), bytes_(std::exchange(o.bytes_, 0)) {}
   DeviceBuffer& operator=(DeviceBuffer&& o) noexcept
   {
      if(this != &o) {
         release();
         p_ = std::exchange(o.p_, nullptr);
         bytes_ = std::exchange(o.bytes_, 0);
      }
      return *this;
   }
   void* get() const noexcept { return p_; }
   std::size_t bytes() const noexcept { return bytes_; }
   void upload(const void* host, std::size_t bytes) const
   {
      if(bytes > bytes_) throw Error(FUFFT_ERR_INVALID, "DeviceBuffer::upload: more bytes than the buffer holds");
      check_hip(hipMemcpy(p_, host, bytes, hipMemcpyHostToDevice), "hipMemcpy");
   }

private:
   void release() noexcept
   {
      if(p_) (void)hipFree(p_);
      p_ = nullptr;
      bytes_ = 0;
   }
   void* p_ = nullptr;
   std::size_t bytes_ = 0;
};

namespace detail {

// Variant::Auto resolved to the fastest variant for a filter layout; an
// unsupported n or layout throws
inline Variant resolve(int64_t n, Variant v, int layout)
{
   if(v != Variant::Auto) return v;
   Variant out = Variant::V16;
   check(fastest_variant(n, &out, layout), "fufft_fastest_variant");
   return out;
}

inline void check_count(int64_t count, const char* where)
{
   if(count < 1) throw Error(FUFFT_ERR_INVALID, std::string(where) + ": filter count must be >= 1");
}

// filt_stride for count filters of `points` points against `batch` items:
// one filter is shared (stride 0), otherwise there must be one per item
inline int64_t stride_for(int64_t count, int64_t batch, int64_t points, const char* where)
{
   if(count == 1) return 0;
   if(batch != count)
      throw Error(FUFFT_ERR_INVALID, std::string(where) + ": batch must equal the plan's filter count");
   return points;
}

}  // namespace detail

// ---- 1D: fufft_pipeline_v16 / _ip / _fused<..., Mid>, the split and BFP calls ---------

// An n-point fused conv with `count` filters (1: shared by the batch; more:
// one per signal, and every launch then takes batch == count).  The filters
// come from the host as taps or natural-order spectra (`kind`) and are
// planned with the 1/n fold, in `layout` (FUFFT_LAYOUT_LANE, the fastest, by
// default) for the variant `v` (Auto: fufft_fastest_variant for that layout).
// The same plan serves the fp32 conv, the int16 BFP conv and the split apply.
template<class Mid = MidMultiply>
class Conv1d {
public:
   Conv1d(int64_t n, const float* natural, int64_t count = 1, int kind = FUFFT_FILTER_TAPS,
          int layout = FUFFT_LAYOUT_LANE, Variant v = Variant::Auto)
      : n_(n), count_(count), layout_(layout), v_(detail::resolve(n, v, layout))
   {
      detail::check_count(count, "Conv1d");
      if(!natural) throw Error(FUFFT_ERR_INVALID, "Conv1d: no filter data");
      std::vector<float> planned(static_cast<std::size_t>(2 * n * count));
      for(int64_t f = 0; f < count; f++)
         check(plan_filter(natural + 2 * n * f, planned.data() + 2 * n * f, n, v_, kind, layout_),
               "fufft_plan_filter_f32");
      filt_ = DeviceBuffer(planned.size() * sizeof(float));
      filt_.upload(planned.data(), planned.size() * sizeof(float));
   }

   // the same plan from filters already in device memory (planned on the
   // device by fufft_plan_filter_device_f32, asynchronously on `stream`)
   static Conv1d from_device(int64_t n, const void* natural, int64_t count = 1, int kind = FUFFT_FILTER_TAPS,
                             int layout = FUFFT_LAYOUT_LANE, Variant v = Variant::Auto, void* stream = nullptr)
   {
      Conv1d c(n, count, layout, detail::resolve(n, v, layout));
      c.filt_ = DeviceBuffer(static_cast<std::size_t>(8 * n * count));
      check(plan_filter_device(natural, c.filt_.get(), n, count, stream, c.v_, kind, layout),
            "fufft_plan_filter_device_f32");
      return c;
   }

   int64_t n() const noexcept { return n_; }
   int64_t count() const noexcept { return count_; }
   Variant variant() const noexcept { return v_; }
   int layout() const noexcept { return layout_; }
   const void* filter() const noexcept { return filt_.get(); }

   // fp32 conv of `batch` signals; in == out is allowed
   void operator()(const void* in, void* out, int64_t batch, void* stream = nullptr) const
   {
      const int64_t st = detail::stride_for(count_, batch, n_, "Conv1d");
      check(pipeline<Mid>(in, filt_.get(), out, n_, batch, stream, st, v_, layout_), "fufft_conv_f32");
   }

   // int16 BFP conv with the same filter: `block`-point blocks, one int8
   // exponent each (fufft_conv_bfp16)
   void bfp(const void* qin, const int8_t* ein, void* qout, int8_t* eout, int64_t batch,
            int64_t block = FUFFT_BFP_BLOCK, void* stream = nullptr) const
   {
      const int64_t st = detail::stride_for(count_, batch, n_, "Conv1d::bfp");
      check(pipeline_bfp<Mid>(qin, ein, filt_.get(), qout, eout, n_, batch, stream, st, v_, layout_, block),
            "fufft_conv_bfp16");
   }

   // the split path: forward spectra (digit order of this plan's variant) ...
   void forward(const void* in, void* spec, int64_t batch, void* stream = nullptr) const
   {
      check(pipeline_fwd(in, spec, n_, batch, stream, v_), "fufft_fwd_f32");
   }

   // ... applied against this plan's filters (spec_stride 0: one spectrum for the batch)
   void apply(const void* spec, int64_t spec_stride, void* out, int64_t batch, void* stream = nullptr) const
   {
      const int64_t st = detail::stride_for(count_, batch, n_, "Conv1d::apply");
      check(pipeline_apply<Mid>(spec, filt_.get(), out, n_, batch, stream, spec_stride, st, v_, layout_),
            "fufft_apply_f32");
   }

private:
   Conv1d(int64_t n, int64_t count, int layout, Variant v) : n_(n), count_(count), layout_(layout), v_(v)
   {
      detail::check_count(count, "Conv1d");
   }
   int64_t n_, count_;
   int layout_;
   Variant v_;
   DeviceBuffer filt_;
};

// ---- int16 BFP in the reference's own format (fufft_pipeline_v16_bfp) ---------------------

// The filter planned in fp32 for (v, layout) and quantised with the
// reference's rule to int16 words and one fp32 scale per filter
// (bfp_quantize, verify_kernel.cpp:1092-1105); signals come with one scale
// per transform (fufft_bfp_scaled_quantize).  Variant::Auto is radix 16, the
// reference's own plan for this kernel.
template<class Mid = MidMultiply>
class ConvBfpScaled {
public:
   ConvBfpScaled(int64_t n, const float* natural, int64_t count = 1, int kind = FUFFT_FILTER_TAPS,
                 int layout = FUFFT_LAYOUT_DR, Variant v = Variant::V16)
      : n_(n), count_(count), layout_(layout), v_(v == Variant::Auto ? Variant::V16 : v)
   {
      detail::check_count(count, "ConvBfpScaled");
      if(!natural) throw Error(FUFFT_ERR_INVALID, "ConvBfpScaled: no filter data");
      std::vector<float> planned(static_cast<std::size_t>(2 * n * count));
      for(int64_t f = 0; f < count; f++)
         check(plan_filter(natural + 2 * n * f, planned.data() + 2 * n * f, n, v_, kind, layout_),
               "fufft_plan_filter_f32");
      std::vector<int16_t> q(planned.size());
      std::vector<float> sc(static_cast<std::size_t>(count));
      check(fufft_bfp_scaled_quantize(planned.data(), n, count, q.data(), sc.data()), "fufft_bfp_scaled_quantize");
      qfilt_ = DeviceBuffer(q.size() * sizeof(int16_t));
      qfilt_.upload(q.data(), q.size() * sizeof(int16_t));
      scale_ = DeviceBuffer(sc.size() * sizeof(float));
      scale_.upload(sc.data(), sc.size() * sizeof(float));
   }

   int64_t n() const noexcept { return n_; }
   Variant variant() const noexcept { return v_; }
   int layout() const noexcept { return layout_; }

   void operator()(const void* qin, const float* sin, void* qout, float* sout, int64_t batch,
                   void* stream = nullptr) const
   {
      const int64_t st = detail::stride_for(count_, batch, n_, "ConvBfpScaled");
      check(pipeline_bfp_scaled<Mid>(qin, sin, qfilt_.get(), static_cast<const float*>(scale_.get()), qout, sout,
                                     n_, batch, stream, st, v_, layout_),
            "fufft_conv_bfp16_scaled");
   }

private:
   int64_t n_, count_;
   int layout_;
   Variant v_;
   DeviceBuffer qfilt_, scale_;
};

// ---- four-step: run_large<N, LOUT, 16, MID, lead, nrv> ----------------------------------------

// The filter in the chain order of the middle `v` picks (Variant::V16, the
// default and Auto: run_large's own V=16 middle, bench_fufft.cu:410-428;
// Variant::R8: the radix-8 middle).  Launches are in place.
template<class Mid = MidMultiply>
class ConvLarge {
public:
   ConvLarge(int64_t n, const float* natural, int64_t count = 1, int kind = FUFFT_FILTER_TAPS,
             Variant v = Variant::V16)
      : n_(n), count_(count), v_(v == Variant::Auto ? Variant::V16 : v)
   {
      detail::check_count(count, "ConvLarge");
      if(!natural) throw Error(FUFFT_ERR_INVALID, "ConvLarge: no filter data");
      check(fufft_large_plan(n, &lout_, &mid_), "fufft_large_plan");
      std::vector<float> planned(static_cast<std::size_t>(2 * n * count));
      for(int64_t f = 0; f < count; f++)
         check(fufft_plan_filter_large_f32(n, (int)v_, kind, 1, natural + 2 * n * f, planned.data() + 2 * n * f),
               "fufft_plan_filter_large_f32");
      filt_ = DeviceBuffer(planned.size() * sizeof(float));
      filt_.upload(planned.data(), planned.size() * sizeof(float));
   }

   int64_t n() const noexcept { return n_; }
   Variant variant() const noexcept { return v_; }
   int outer_levels() const noexcept { return lout_; }
   int middle() const noexcept { return mid_; }
   const void* filter() const noexcept { return filt_.get(); }

   void operator()(void* buf, int64_t batch, void* stream = nullptr) const
   {
      const int64_t st = detail::stride_for(count_, batch, n_, "ConvLarge");
      check(fufft_conv_large_f32(buf, filt_.get(), st, n_, batch, Mid::id, (int)v_, stream), "fufft_conv_large_f32");
   }

private:
   int64_t n_, count_;
   Variant v_;
   int lout_ = 0, mid_ = 0;
   DeviceBuffer filt_;
};

// ---- 2D: fufft_conv2d<H, W, CPB>, the two-for-one real and split calls --------------------

// An h x w image conv; the filter planned in `layout` (FUFFT_LAYOUT_LANE, the
// library's column order, by default; FUFFT_LAYOUT_DR the reference's).
template<class Mid = MidMultiply>
class Conv2d {
public:
   Conv2d(int64_t h, int64_t w, const float* natural, int64_t count = 1, int kind = FUFFT_FILTER_TAPS,
          int layout = FUFFT_LAYOUT_LANE)
      : h_(h), w_(w), count_(count), layout_(layout)
   {
      detail::check_count(count, "Conv2d");
      if(!natural) throw Error(FUFFT_ERR_INVALID, "Conv2d: no filter data");
      const int64_t np = h * w;
      std::vector<float> planned(static_cast<std::size_t>(2 * np * count));
      for(int64_t f = 0; f < count; f++)
         check(fufft_plan_filter2d_f32(h, w, layout_, kind, 1, natural + 2 * np * f, planned.data() + 2 * np * f),
               "fufft_plan_filter2d_f32");
      filt_ = DeviceBuffer(planned.size() * sizeof(float));
      filt_.upload(planned.data(), planned.size() * sizeof(float));
   }

   int64_t height() const noexcept { return h_; }
   int64_t width() const noexcept { return w_; }
   int layout() const noexcept { return layout_; }
   const void* filter() const noexcept { return filt_.get(); }

   void operator()(const void* in, void* out, int64_t batch, void* stream = nullptr) const
   {
      const int64_t st = detail::stride_for(count_, batch, h_ * w_, "Conv2d");
      check(fufft_conv2d_f32(in, filt_.get(), st, out, h_, w_, batch, Mid::id, layout_, stream), "fufft_conv2d_f32");
   }

   // two real images per complex transform (x + iy); correct for a filter of
   // real taps; `work` holds batch * h * w complex points
   void real2(const float* x, const float* y, float* u, float* v, void* work, int64_t batch,
              void* stream = nullptr) const
   {
      const int64_t st = detail::stride_for(count_, batch, h_ * w_, "Conv2d::real2");
      check(fufft_conv2d_r2_f32(x, y, filt_.get(), st, u, v, work, h_, w_, batch, layout_, stream),
            "fufft_conv2d_r2_f32");
   }

   // the split path: 2D spectra of `batch` images, then those (or one, spec_stride 0)
   // applied against this plan's filters
   void forward(const void* in, void* spec, int64_t batch, void* stream = nullptr) const
   {
      check(fufft_fwd2d_f32(in, spec, h_, w_, batch, stream), "fufft_fwd2d_f32");
   }
   void apply(const void* spec, int64_t spec_stride, void* out, int64_t batch, void* stream = nullptr) const
   {
      const int64_t st = detail::stride_for(count_, batch, h_ * w_, "Conv2d::apply");
      check(fufft_apply2d_f32(spec, spec_stride, filt_.get(), st, out, h_, w_, batch, Mid::id, layout_, stream),
            "fufft_apply2d_f32");
   }

private:
   int64_t h_, w_, count_;
   int layout_;
   DeviceBuffer filt_;
};

}  // namespace fufft

#endif  // FUFFT_PLAN_HPP
