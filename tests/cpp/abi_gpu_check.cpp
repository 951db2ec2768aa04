// A C++ caller of the library on the GPU, with no Python anywhere: the HIP
// runtime for memory and streams, include/fufft/fufft.hpp for the calls.
// It convolves a seeded batch at N = 4096 (FUFFT_AUTO) three ways and checks:
//   - fufft::pipeline<MidMultiply> against an fp64 direct cyclic convolution
//     (O(N^2) per checked signal), rel L2 <= 2e-6;
//   - the raw C entry point fufft_conv_f32 bit for bit against the template;
//   - in place (in == out) bit for bit against out of place;
//   - the split path (pipeline_fwd + pipeline_apply) bit for bit against fused;
//   - the int16 BFP conv in the reference's own format (pipeline_bfp_scaled:
//     fp32 scale per transform, int16 filter) bit for bit against its
//     definition: dequantise on the host, the fp32 conv on the GPU, quantise
//     on the host with the same codec (fufft_bfp_scaled_*);
//   - a small 2D image (64 x 64, one fused launch) against an fp64 direct 2D
//     cyclic convolution, rel L2 <= 2e-6;
//   - the plan objects of include/fufft/plan.hpp (Conv1d with the lane-major
//     filter at the fastest variant and with the reference's digit order,
//     Conv1d::from_device, the BFP conv through a Conv1d, ConvLarge with the
//     reference's V=16 middle, Conv2d, and a Conv1d at N = 32768, the
//     single-launch 32-values-per-lane conv) bit for bit against the C calls
//     with filters planned by hand, and their argument errors as fufft::Error;
//   - the reference's launch surface by name (fufft::ref: fufft_pipeline_v16,
//     _ip, _v16f, _fwd / _apply, _v16_bfp, run_large) with one filter per
//     transform, bit for bit against the C calls, and run_large refusing a
//     split the library does not run.
// Built by fufft_amd/build.py into tests/cpp/_build/abi_gpu_check and run by
// tests/test_gpu_cpp_caller.py.  Prints "ok ..." and returns 0 on success.
#include "fufft/fufft.hpp"
#include "fufft/plan.hpp"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

namespace {

#define CHECK_HIP(x)                                                                        \
   do {                                                                                     \
      const hipError_t e_ = (x);                                                            \
      if(e_ != hipSuccess) {                                                                \
         std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
         return 10;                                                                         \
      }                                                                                     \
   } while(0)

#define CHECK_FU(x)                                                                         \
   do {                                                                                     \
      const int s_ = (x);                                                                   \
      if(s_ != FUFFT_OK) {                                                                  \
         std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, fufft::status_string(s_)); \
         return 11;                                                                         \
      }                                                                                     \
   } while(0)

// xorshift64*: a seeded, platform-independent uniform in [-1, 1)
struct Rng {
   uint64_t s;
   float next()
   {
      s ^= s >> 12; s ^= s << 25; s ^= s >> 27;
      const uint64_t r = s * 0x2545F4914F6CDD1Dull;
      return (float)((double)(r >> 11) * (1.0 / 9007199254740992.0) * 2.0 - 1.0);
   }
};

bool same_bits(const std::vector<float>& a, const std::vector<float>& b)
{
   return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0;
}

}  // namespace

int main()
{
   const int64_t n = 4096, batch = 16;
   const size_t pts = (size_t)(n * batch);
   Rng rng{0x5eedf00dull};
   std::vector<float> a(2 * pts), taps(2 * n), filt(2 * n);
   for(auto& x : a) x = rng.next();
   for(auto& x : taps) x = rng.next();

   CHECK_FU(fufft::init(0));
   CHECK_FU(fufft::plan_filter(taps.data(), filt.data(), n));        // FUFFT_AUTO, taps, 1/n folded

   hipStream_t s;
   CHECK_HIP(hipStreamCreate(&s));
   void *d_a = nullptr, *d_f = nullptr, *d_o = nullptr, *d_o2 = nullptr, *d_spec = nullptr;
   CHECK_HIP(hipMalloc(&d_a, pts * 8));
   CHECK_HIP(hipMalloc(&d_f, (size_t)n * 8));
   CHECK_HIP(hipMalloc(&d_o, pts * 8));
   CHECK_HIP(hipMalloc(&d_o2, pts * 8));
   CHECK_HIP(hipMalloc(&d_spec, pts * 8));
   CHECK_HIP(hipMemcpy(d_a, a.data(), pts * 8, hipMemcpyHostToDevice));
   CHECK_HIP(hipMemcpy(d_f, filt.data(), (size_t)n * 8, hipMemcpyHostToDevice));

   // 1. the template surface
   CHECK_FU(fufft::pipeline<fufft::MidMultiply>(d_a, d_f, d_o, n, batch, s));
   std::vector<float> out(2 * pts), out2(2 * pts);
   CHECK_HIP(hipStreamSynchronize(s));
   CHECK_HIP(hipMemcpy(out.data(), d_o, pts * 8, hipMemcpyDeviceToHost));

   // 2. the raw C entry point, same arguments
   CHECK_FU(fufft_conv_f32(d_a, d_f, 0, d_o2, n, batch, FUFFT_MID_MUL, FUFFT_AUTO, FUFFT_LAYOUT_DR, s));
   CHECK_HIP(hipStreamSynchronize(s));
   CHECK_HIP(hipMemcpy(out2.data(), d_o2, pts * 8, hipMemcpyDeviceToHost));
   if(!same_bits(out, out2)) { std::fprintf(stderr, "C entry point differs from the template\n"); return 2; }

   // 3. split forward + apply against fused
   CHECK_FU(fufft::pipeline_fwd(d_a, d_spec, n, batch, s));
   CHECK_FU(fufft::pipeline_apply<fufft::MidMultiply>(d_spec, d_f, d_o2, n, batch, s, /*spec_stride=*/n));
   CHECK_HIP(hipStreamSynchronize(s));
   CHECK_HIP(hipMemcpy(out2.data(), d_o2, pts * 8, hipMemcpyDeviceToHost));
   if(!same_bits(out, out2)) { std::fprintf(stderr, "split path differs from fused\n"); return 3; }

   // 4. in place
   CHECK_FU(fufft::pipeline<fufft::MidMultiply>(d_a, d_f, d_a, n, batch, s));
   CHECK_HIP(hipStreamSynchronize(s));
   CHECK_HIP(hipMemcpy(out2.data(), d_a, pts * 8, hipMemcpyDeviceToHost));
   if(!same_bits(out, out2)) { std::fprintf(stderr, "in place differs from out of place\n"); return 4; }

   // 5. fp64 direct cyclic convolution y[k] = sum_i a[i] b[(k - i) mod n] on two signals
   double num = 0.0, den = 0.0;
   for(int64_t sig : {int64_t(0), batch - 1}) {
      const float* x = a.data() + 2 * sig * n;
      for(int64_t k = 0; k < n; k++) {
         double re = 0.0, im = 0.0;
         for(int64_t i = 0; i < n; i++) {
            const int64_t j = (k - i + n) % n;
            const double ar = x[2 * i], ai = x[2 * i + 1], br = taps[2 * j], bi = taps[2 * j + 1];
            re += ar * br - ai * bi;
            im += ar * bi + ai * br;
         }
         const double gr = out[2 * (sig * n + k)], gi = out[2 * (sig * n + k) + 1];
         num += (gr - re) * (gr - re) + (gi - im) * (gi - im);
         den += re * re + im * im;
      }
   }
   const double rel = std::sqrt(num / den);
   if(!(rel <= 2e-6)) { std::fprintf(stderr, "rel L2 vs fp64 direct %.3e > 2e-6\n", rel); return 5; }

   // 6. int16 BFP in the reference's format, radix 16 (its plan): the words and
   //    scales equal quantise(conv(dequantise(signal), dequantise(filter)))
   {
      std::vector<float> fv(2 * n);
      CHECK_FU(fufft::plan_filter(taps.data(), fv.data(), n, fufft::Variant::V16));
      std::vector<int16_t> q(2 * pts), fq(2 * n), qo(2 * pts), wq(2 * pts);
      std::vector<float> sc(batch), fs(1), so(batch), ws(batch), ad(2 * pts), fd(2 * n), y(2 * pts);
      CHECK_FU(fufft_bfp_scaled_quantize(a.data(), n, batch, q.data(), sc.data()));
      CHECK_FU(fufft_bfp_scaled_quantize(fv.data(), n, 1, fq.data(), fs.data()));
      CHECK_FU(fufft_bfp_scaled_dequantize(q.data(), sc.data(), n, batch, ad.data()));
      CHECK_FU(fufft_bfp_scaled_dequantize(fq.data(), fs.data(), n, 1, fd.data()));
      void *d_q = nullptr, *d_fq = nullptr;
      float *d_s = nullptr, *d_fs = nullptr, *d_so = nullptr;
      CHECK_HIP(hipMalloc(&d_q, pts * 4)); CHECK_HIP(hipMalloc(&d_fq, (size_t)n * 4));
      CHECK_HIP(hipMalloc(&d_s, batch * 4)); CHECK_HIP(hipMalloc(&d_fs, 4)); CHECK_HIP(hipMalloc(&d_so, batch * 4));
      CHECK_HIP(hipMemcpy(d_q, q.data(), pts * 4, hipMemcpyHostToDevice));
      CHECK_HIP(hipMemcpy(d_fq, fq.data(), (size_t)n * 4, hipMemcpyHostToDevice));
      CHECK_HIP(hipMemcpy(d_s, sc.data(), batch * 4, hipMemcpyHostToDevice));
      CHECK_HIP(hipMemcpy(d_fs, fs.data(), 4, hipMemcpyHostToDevice));
      CHECK_FU(fufft::pipeline_bfp_scaled<fufft::MidMultiply>(d_q, d_s, d_fq, d_fs, d_q, d_so, n, batch, s));
      CHECK_HIP(hipMemcpy(d_o2, ad.data(), pts * 8, hipMemcpyHostToDevice));
      CHECK_HIP(hipMemcpy(d_f, fd.data(), (size_t)n * 8, hipMemcpyHostToDevice));
      CHECK_FU(fufft::pipeline<fufft::MidMultiply>(d_o2, d_f, d_o2, n, batch, s, 0, fufft::Variant::V16));
      CHECK_HIP(hipStreamSynchronize(s));
      CHECK_HIP(hipMemcpy(qo.data(), d_q, pts * 4, hipMemcpyDeviceToHost));
      CHECK_HIP(hipMemcpy(so.data(), d_so, batch * 4, hipMemcpyDeviceToHost));
      CHECK_HIP(hipMemcpy(y.data(), d_o2, pts * 8, hipMemcpyDeviceToHost));
      CHECK_FU(fufft_bfp_scaled_quantize(y.data(), n, batch, wq.data(), ws.data()));
      if(std::memcmp(qo.data(), wq.data(), qo.size() * 2) != 0 || std::memcmp(so.data(), ws.data(), so.size() * 4) != 0) {
         std::fprintf(stderr, "reference-format BFP differs from dequantise -> conv -> quantise\n");
         return 6;
      }
      CHECK_HIP(hipFree(d_q)); CHECK_HIP(hipFree(d_fq)); CHECK_HIP(hipFree(d_s)); CHECK_HIP(hipFree(d_fs));
      CHECK_HIP(hipFree(d_so));
   }

   // 7. a small image in one fused launch against an fp64 direct 2D cyclic convolution
   double rel2 = 0.0;
   {
      const int64_t h = 64, w = 64, np = h * w, nimg = 3;
      std::vector<float> img(2 * np * nimg), t2(2 * np), f2(2 * np), o2(2 * np * nimg);
      for(auto& x : img) x = rng.next();
      for(auto& x : t2) x = rng.next();
      CHECK_FU(fufft_plan_filter2d_f32(h, w, FUFFT_LAYOUT_DR, FUFFT_FILTER_TAPS, 1, t2.data(), f2.data()));
      CHECK_HIP(hipMemcpy(d_o, img.data(), np * nimg * 8, hipMemcpyHostToDevice));
      CHECK_HIP(hipMemcpy(d_f, f2.data(), np * 8, hipMemcpyHostToDevice));
      CHECK_FU(fufft_conv2d_f32(d_o, d_f, 0, d_o2, h, w, nimg, FUFFT_MID_MUL, FUFFT_LAYOUT_DR, s));
      CHECK_HIP(hipStreamSynchronize(s));
      CHECK_HIP(hipMemcpy(o2.data(), d_o2, np * nimg * 8, hipMemcpyDeviceToHost));
      double num2 = 0.0, den2 = 0.0;
      const int64_t im = nimg - 1;
      for(int64_t r = 0; r < h; r++)
         for(int64_t c = 0; c < w; c++) {
            double re = 0.0, iv = 0.0;
            for(int64_t i = 0; i < h; i++)
               for(int64_t j = 0; j < w; j++) {
                  const int64_t ti = ((r - i + h) % h) * w + (c - j + w) % w;
                  const double ar = img[2 * (im * np + i * w + j)], ai = img[2 * (im * np + i * w + j) + 1];
                  re += ar * t2[2 * ti] - ai * t2[2 * ti + 1];
                  iv += ar * t2[2 * ti + 1] + ai * t2[2 * ti];
               }
            const double gr = o2[2 * (im * np + r * w + c)], gi = o2[2 * (im * np + r * w + c) + 1];
            num2 += (gr - re) * (gr - re) + (gi - iv) * (gi - iv);
            den2 += re * re + iv * iv;
         }
      rel2 = std::sqrt(num2 / den2);
      if(!(rel2 <= 2e-6)) { std::fprintf(stderr, "2D rel L2 vs fp64 direct %.3e > 2e-6\n", rel2); return 7; }
   }

   // 8. plan objects against the C calls they make, on fresh input
   int plans = 0;
   try {
      std::vector<float> x(2 * pts), want(2 * pts), got(2 * pts), fl(2 * n);
      for(auto& v : x) v = rng.next();
      CHECK_HIP(hipMemcpy(d_a, x.data(), pts * 8, hipMemcpyHostToDevice));
      // (a) the fastest plan: lane-major filter at fufft_fastest_variant's variant
      fufft::Conv1d<fufft::MidMultiply> fast(n, taps.data());
      fufft::Variant fv = fufft::Variant::Auto;
      CHECK_FU(fufft::fastest_variant(n, &fv, FUFFT_LAYOUT_LANE));
      if(fast.variant() != fv || fast.layout() != FUFFT_LAYOUT_LANE) { std::fprintf(stderr, "Conv1d plan\n"); return 20; }
      CHECK_FU(fufft::plan_filter(taps.data(), fl.data(), n, fv, FUFFT_FILTER_TAPS, FUFFT_LAYOUT_LANE));
      CHECK_HIP(hipMemcpy(d_f, fl.data(), (size_t)n * 8, hipMemcpyHostToDevice));
      CHECK_FU(fufft::pipeline<fufft::MidMultiply>(d_a, d_f, d_o, n, batch, s, 0, fv, FUFFT_LAYOUT_LANE));
      fast(d_a, d_o2, batch, s);
      CHECK_HIP(hipStreamSynchronize(s));
      CHECK_HIP(hipMemcpy(want.data(), d_o, pts * 8, hipMemcpyDeviceToHost));
      CHECK_HIP(hipMemcpy(got.data(), d_o2, pts * 8, hipMemcpyDeviceToHost));
      if(!same_bits(want, got)) { std::fprintf(stderr, "Conv1d (lane) differs from the C call\n"); return 21; }
      plans++;
      // (b) the reference's own plan and filter order
      fufft::Conv1d<fufft::MidMultiply> ref(n, taps.data(), 1, FUFFT_FILTER_TAPS, FUFFT_LAYOUT_DR, fufft::Variant::V16);
      CHECK_FU(fufft::plan_filter(taps.data(), fl.data(), n, fufft::Variant::V16));
      CHECK_HIP(hipMemcpy(d_f, fl.data(), (size_t)n * 8, hipMemcpyHostToDevice));
      CHECK_FU(fufft::pipeline<fufft::MidMultiply>(d_a, d_f, d_o, n, batch, s, 0, fufft::Variant::V16));
      ref(d_a, d_o2, batch, s);
      CHECK_HIP(hipStreamSynchronize(s));
      CHECK_HIP(hipMemcpy(want.data(), d_o, pts * 8, hipMemcpyDeviceToHost));
      CHECK_HIP(hipMemcpy(got.data(), d_o2, pts * 8, hipMemcpyDeviceToHost));
      if(!same_bits(want, got)) { std::fprintf(stderr, "Conv1d (digit order, V16) differs\n"); return 22; }
      plans++;
      // (c) one filter per signal, planned on the device from natural-order
      //     spectra, against the same spectra planned on the host
      {
         const int64_t cnt = batch;
         std::vector<float> specs(2 * pts);
         for(auto& v : specs) v = rng.next();
         fufft::Conv1d<fufft::MidConjMultiply> host(n, specs.data(), cnt, FUFFT_FILTER_SPECTRUM);
         CHECK_HIP(hipMemcpy(d_spec, specs.data(), pts * 8, hipMemcpyHostToDevice));
         auto dev = fufft::Conv1d<fufft::MidConjMultiply>::from_device(n, d_spec, cnt, FUFFT_FILTER_SPECTRUM,
                                                                      FUFFT_LAYOUT_LANE, fufft::Variant::Auto, s);
         host(d_a, d_o, batch, s);
         dev(d_a, d_o2, batch, s);
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(want.data(), d_o, pts * 8, hipMemcpyDeviceToHost));
         CHECK_HIP(hipMemcpy(got.data(), d_o2, pts * 8, hipMemcpyDeviceToHost));
         if(!same_bits(want, got)) { std::fprintf(stderr, "Conv1d::from_device differs from the host plan\n"); return 23; }
         // a per-signal plan refuses a batch of another size
         bool threw = false;
         try {
            host(d_a, d_o, batch - 1, s);
         } catch(const fufft::Error& e) {
            threw = e.status() == FUFFT_ERR_INVALID;
         }
         if(!threw) { std::fprintf(stderr, "per-signal plan accepted a mismatched batch\n"); return 24; }
         plans++;
      }
      // (d) the BFP conv through the same plan as the fp32 conv
      {
         std::vector<int16_t> q(2 * pts), qa(2 * pts), qb(2 * pts);
         std::vector<int8_t> e(pts / 64), ea(pts / 64), eb(pts / 64);
         CHECK_FU(fufft_bfp_quantize(x.data(), (int64_t)pts, 64, q.data(), e.data()));
         void *d_q = nullptr, *d_qo = nullptr, *d_e = nullptr, *d_eo = nullptr;
         CHECK_HIP(hipMalloc(&d_q, pts * 4)); CHECK_HIP(hipMalloc(&d_qo, pts * 4));
         CHECK_HIP(hipMalloc(&d_e, pts / 64)); CHECK_HIP(hipMalloc(&d_eo, pts / 64));
         CHECK_HIP(hipMemcpy(d_q, q.data(), pts * 4, hipMemcpyHostToDevice));
         CHECK_HIP(hipMemcpy(d_e, e.data(), pts / 64, hipMemcpyHostToDevice));
         CHECK_FU(fufft::plan_filter(taps.data(), fl.data(), n, fv, FUFFT_FILTER_TAPS, FUFFT_LAYOUT_LANE));
         CHECK_HIP(hipMemcpy(d_f, fl.data(), (size_t)n * 8, hipMemcpyHostToDevice));
         CHECK_FU(fufft::pipeline_bfp<fufft::MidMultiply>(d_q, static_cast<int8_t*>(d_e), d_f, d_qo,
                                                         static_cast<int8_t*>(d_eo), n, batch, s, 0, fv,
                                                         FUFFT_LAYOUT_LANE));
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(qa.data(), d_qo, pts * 4, hipMemcpyDeviceToHost));
         CHECK_HIP(hipMemcpy(ea.data(), d_eo, pts / 64, hipMemcpyDeviceToHost));
         fast.bfp(d_q, static_cast<int8_t*>(d_e), d_qo, static_cast<int8_t*>(d_eo), batch, 64, s);
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(qb.data(), d_qo, pts * 4, hipMemcpyDeviceToHost));
         CHECK_HIP(hipMemcpy(eb.data(), d_eo, pts / 64, hipMemcpyDeviceToHost));
         CHECK_HIP(hipFree(d_q)); CHECK_HIP(hipFree(d_qo)); CHECK_HIP(hipFree(d_e)); CHECK_HIP(hipFree(d_eo));
         if(std::memcmp(qa.data(), qb.data(), qa.size() * 2) != 0 || std::memcmp(ea.data(), eb.data(), ea.size()) != 0) {
            std::fprintf(stderr, "Conv1d::bfp differs from the C call\n");
            return 25;
         }
         plans++;
      }
      // (e) four-step with the reference's V=16 middle, in place
      {
         const int64_t nl = 32768, bl = 2;
         std::vector<float> tl(2 * nl), fl2(2 * nl), xl(2 * nl * bl), a1(2 * nl * bl), a2(2 * nl * bl);
         for(auto& v : tl) v = rng.next();
         for(auto& v : xl) v = rng.next();
         fufft::ConvLarge<fufft::MidMultiply> large(nl, tl.data());
         if(large.variant() != fufft::Variant::V16 || large.outer_levels() != 1 || large.middle() != 2048) {
            std::fprintf(stderr, "ConvLarge plan\n");
            return 26;
         }
         CHECK_FU(fufft_plan_filter_large_f32(nl, FUFFT_V16, FUFFT_FILTER_TAPS, 1, tl.data(), fl2.data()));
         void* d_l = nullptr; void* d_lf = nullptr;
         CHECK_HIP(hipMalloc(&d_l, (size_t)nl * bl * 8)); CHECK_HIP(hipMalloc(&d_lf, (size_t)nl * 8));
         CHECK_HIP(hipMemcpy(d_lf, fl2.data(), (size_t)nl * 8, hipMemcpyHostToDevice));
         CHECK_HIP(hipMemcpy(d_l, xl.data(), (size_t)nl * bl * 8, hipMemcpyHostToDevice));
         CHECK_FU(fufft_conv_large_f32(d_l, d_lf, 0, nl, bl, FUFFT_MID_MUL, FUFFT_V16, s));
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(a1.data(), d_l, (size_t)nl * bl * 8, hipMemcpyDeviceToHost));
         CHECK_HIP(hipMemcpy(d_l, xl.data(), (size_t)nl * bl * 8, hipMemcpyHostToDevice));
         large(d_l, bl, s);
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(a2.data(), d_l, (size_t)nl * bl * 8, hipMemcpyDeviceToHost));
         CHECK_HIP(hipFree(d_l)); CHECK_HIP(hipFree(d_lf));
         if(!same_bits(a1, a2)) { std::fprintf(stderr, "ConvLarge differs from the C call\n"); return 27; }
         plans++;
      }
      // (f) 2D, 64 x 64 (its column order is the identity: both layouts give the same filter)
      {
         const int64_t h = 64, w = 64, np = h * w, nimg = 3;
         std::vector<float> img(2 * np * nimg), t2(2 * np), f2(2 * np), b1(2 * np * nimg), b2(2 * np * nimg);
         for(auto& v : img) v = rng.next();
         for(auto& v : t2) v = rng.next();
         fufft::Conv2d<fufft::MidMultiply> c2(h, w, t2.data());
         CHECK_FU(fufft_plan_filter2d_f32(h, w, FUFFT_LAYOUT_LANE, FUFFT_FILTER_TAPS, 1, t2.data(), f2.data()));
         CHECK_HIP(hipMemcpy(d_a, img.data(), np * nimg * 8, hipMemcpyHostToDevice));
         CHECK_HIP(hipMemcpy(d_f, f2.data(), np * 8, hipMemcpyHostToDevice));
         CHECK_FU(fufft_conv2d_f32(d_a, d_f, 0, d_o, h, w, nimg, FUFFT_MID_MUL, FUFFT_LAYOUT_LANE, s));
         c2(d_a, d_o2, nimg, s);
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(b1.data(), d_o, np * nimg * 8, hipMemcpyDeviceToHost));
         CHECK_HIP(hipMemcpy(b2.data(), d_o2, np * nimg * 8, hipMemcpyDeviceToHost));
         if(!same_bits(b1, b2)) { std::fprintf(stderr, "Conv2d differs from the C call\n"); return 28; }
         plans++;
      }
      // (g) N = 32768 in one launch: a Conv1d at its fastest plan (lane-major
      //     filter) against the C call with the digit-order filter, bit for
      //     bit (the same plan and arithmetic, another filter layout)
      {
         const int64_t nw = 32768, bw = 3;
         std::vector<float> xw(2 * nw * bw), tw(2 * nw), fw(2 * nw), w1(2 * nw * bw), w2(2 * nw * bw);
         for(auto& v : xw) v = rng.next();
         for(auto& v : tw) v = rng.next();
         fufft::Conv1d<fufft::MidMultiply> wide(nw, tw.data());
         if(wide.variant() != fufft::Variant::V16 || wide.layout() != FUFFT_LAYOUT_LANE) {
            std::fprintf(stderr, "Conv1d plan at N = 32768\n");
            return 30;
         }
         CHECK_FU(fufft::plan_filter(tw.data(), fw.data(), nw, fufft::Variant::V16, FUFFT_FILTER_TAPS, FUFFT_LAYOUT_DR));
         void* d_w = nullptr; void* d_wf = nullptr; void* d_wo = nullptr;
         CHECK_HIP(hipMalloc(&d_w, (size_t)nw * bw * 8)); CHECK_HIP(hipMalloc(&d_wf, (size_t)nw * 8));
         CHECK_HIP(hipMalloc(&d_wo, (size_t)nw * bw * 8));
         CHECK_HIP(hipMemcpy(d_w, xw.data(), (size_t)nw * bw * 8, hipMemcpyHostToDevice));
         CHECK_HIP(hipMemcpy(d_wf, fw.data(), (size_t)nw * 8, hipMemcpyHostToDevice));
         CHECK_FU(fufft_conv_f32(d_w, d_wf, 0, d_wo, nw, bw, FUFFT_MID_MUL, FUFFT_V16, FUFFT_LAYOUT_DR, s));
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(w1.data(), d_wo, (size_t)nw * bw * 8, hipMemcpyDeviceToHost));
         wide(d_w, d_wo, bw, s);
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(w2.data(), d_wo, (size_t)nw * bw * 8, hipMemcpyDeviceToHost));
         CHECK_HIP(hipFree(d_w)); CHECK_HIP(hipFree(d_wf)); CHECK_HIP(hipFree(d_wo));
         if(!same_bits(w1, w2)) { std::fprintf(stderr, "Conv1d at N = 32768 differs from the C call\n"); return 31; }
         plans++;
      }
   } catch(const fufft::Error& e) {
      std::fprintf(stderr, "plan object: %s\n", e.what());
      return 29;
   }

   // 9. the reference's launch surface by name (fufft::ref), one filter per
   //    transform as its kernels read them, against the C calls
   int refs = 0;
   {
      std::vector<float> x(2 * pts), tb(2 * pts), f16(2 * pts), f8(2 * pts), fbp(2 * pts), want(2 * pts), got(2 * pts);
      for(auto& v : x) v = rng.next();
      for(auto& v : tb) v = rng.next();
      for(int64_t t = 0; t < batch; t++) {
         CHECK_FU(fufft::plan_filter(tb.data() + 2 * t * n, f16.data() + 2 * t * n, n, fufft::Variant::V16));
         CHECK_FU(fufft::plan_filter(tb.data() + 2 * t * n, f8.data() + 2 * t * n, n, fufft::Variant::R8));
         CHECK_FU(fufft::plan_filter(tb.data() + 2 * t * n, fbp.data() + 2 * t * n, n, fufft::Variant::V16,
                                     FUFFT_FILTER_TAPS, FUFFT_LAYOUT_BPERM));
      }
      void *d_f16 = nullptr, *d_f8 = nullptr, *d_fbp = nullptr;
      CHECK_HIP(hipMalloc(&d_f16, pts * 8)); CHECK_HIP(hipMalloc(&d_f8, pts * 8)); CHECK_HIP(hipMalloc(&d_fbp, pts * 8));
      CHECK_HIP(hipMemcpy(d_a, x.data(), pts * 8, hipMemcpyHostToDevice));
      CHECK_HIP(hipMemcpy(d_f16, f16.data(), pts * 8, hipMemcpyHostToDevice));
      CHECK_HIP(hipMemcpy(d_f8, f8.data(), pts * 8, hipMemcpyHostToDevice));
      CHECK_HIP(hipMemcpy(d_fbp, fbp.data(), pts * 8, hipMemcpyHostToDevice));
      // 0 when d_o and d_o2 hold the same bits, else `code` (10 on a HIP error)
      auto compare = [&](const char* what, int code) -> int {
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(want.data(), d_o, pts * 8, hipMemcpyDeviceToHost));
         CHECK_HIP(hipMemcpy(got.data(), d_o2, pts * 8, hipMemcpyDeviceToHost));
         if(!same_bits(want, got)) { std::fprintf(stderr, "fufft::ref::%s differs from the C call\n", what); return code; }
         refs++;
         return 0;
      };
      // fufft_pipeline_v16<N, LEAD, NRV, CPB> with MidMultiply{b}
      CHECK_FU(fufft_conv_f32(d_a, d_f16, n, d_o, n, batch, FUFFT_MID_MUL, FUFFT_V16, FUFFT_LAYOUT_DR, s));
      CHECK_FU((fufft::ref::fufft_pipeline_v16<4096, 1, 3, 1>(d_a, d_o2, fufft::MidMultiply{d_f16}, batch, s)));
      if(const int r = compare("fufft_pipeline_v16", 40)) return r;
      // fufft_pipeline_ip<N, LEAD, NR8, CPB, Mid> with a correlation
      CHECK_FU(fufft_conv_f32(d_a, d_f8, n, d_o, n, batch, FUFFT_MID_CONJ, FUFFT_R8, FUFFT_LAYOUT_DR, s));
      CHECK_FU((fufft::ref::fufft_pipeline_ip<4096, 1, 4, 8, fufft::MidConjMultiply>(
         d_a, d_o2, fufft::MidConjMultiply{d_f8}, batch, s)));
      if(const int r = compare("fufft_pipeline_ip", 41)) return r;
      // fufft_pipeline_v16f<N, LEAD, NRV, CPB> with the bperm filter: the same
      // results as fufft_pipeline_v16 with the digit-order one
      CHECK_FU(fufft_conv_f32(d_a, d_f16, n, d_o, n, batch, FUFFT_MID_MUL, FUFFT_V16, FUFFT_LAYOUT_DR, s));
      CHECK_FU((fufft::ref::fufft_pipeline_v16f<4096, 1, 3, 1>(d_a, d_fbp, d_o2, batch, s)));
      if(const int r = compare("fufft_pipeline_v16f", 42)) return r;
      // fufft_pipeline_fwd + fufft_pipeline_apply (radix 8) against fufft_pipeline_ip
      CHECK_FU((fufft::ref::fufft_pipeline_ip<4096, 1, 4, 8, fufft::MidMultiply>(
         d_a, d_o, fufft::MidMultiply{d_f8}, batch, s)));
      CHECK_FU((fufft::ref::fufft_pipeline_fwd<4096, 1, 4, 8>(d_a, d_spec, batch, s)));
      CHECK_FU((fufft::ref::fufft_pipeline_apply<4096, 1, 4, 8>(d_spec, d_f8, d_o2, batch, s)));
      if(const int r = compare("fufft_pipeline_fwd / _apply", 43)) return r;
      // fufft_pipeline_v16_bfp<N, LEAD, NRV, CPB>: int16 filter and scale per transform
      {
         std::vector<int16_t> q(2 * pts), fq(2 * pts), q1(2 * pts), q2(2 * pts);
         std::vector<float> sc(batch), fs(batch), s1(batch), s2(batch);
         CHECK_FU(fufft_bfp_scaled_quantize(x.data(), n, batch, q.data(), sc.data()));
         CHECK_FU(fufft_bfp_scaled_quantize(f16.data(), n, batch, fq.data(), fs.data()));
         void *d_q = nullptr, *d_fq = nullptr, *d_qo = nullptr;
         float *d_s = nullptr, *d_fs = nullptr, *d_so = nullptr;
         CHECK_HIP(hipMalloc(&d_q, pts * 4)); CHECK_HIP(hipMalloc(&d_fq, pts * 4)); CHECK_HIP(hipMalloc(&d_qo, pts * 4));
         CHECK_HIP(hipMalloc(&d_s, batch * 4)); CHECK_HIP(hipMalloc(&d_fs, batch * 4)); CHECK_HIP(hipMalloc(&d_so, batch * 4));
         CHECK_HIP(hipMemcpy(d_q, q.data(), pts * 4, hipMemcpyHostToDevice));
         CHECK_HIP(hipMemcpy(d_fq, fq.data(), pts * 4, hipMemcpyHostToDevice));
         CHECK_HIP(hipMemcpy(d_s, sc.data(), batch * 4, hipMemcpyHostToDevice));
         CHECK_HIP(hipMemcpy(d_fs, fs.data(), batch * 4, hipMemcpyHostToDevice));
         CHECK_FU(fufft_conv_bfp16_scaled(d_q, d_s, d_fq, d_fs, n, d_qo, d_so, n, batch, FUFFT_MID_MUL, FUFFT_V16,
                                          FUFFT_LAYOUT_DR, s));
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(q1.data(), d_qo, pts * 4, hipMemcpyDeviceToHost));
         CHECK_HIP(hipMemcpy(s1.data(), d_so, batch * 4, hipMemcpyDeviceToHost));
         CHECK_FU((fufft::ref::fufft_pipeline_v16_bfp<4096, 1, 3, 1>(d_q, d_s, d_fq, d_fs, d_qo, d_so, batch, s)));
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(q2.data(), d_qo, pts * 4, hipMemcpyDeviceToHost));
         CHECK_HIP(hipMemcpy(s2.data(), d_so, batch * 4, hipMemcpyDeviceToHost));
         CHECK_HIP(hipFree(d_q)); CHECK_HIP(hipFree(d_fq)); CHECK_HIP(hipFree(d_qo));
         CHECK_HIP(hipFree(d_s)); CHECK_HIP(hipFree(d_fs)); CHECK_HIP(hipFree(d_so));
         if(std::memcmp(q1.data(), q2.data(), q1.size() * 2) != 0 || std::memcmp(s1.data(), s2.data(), s1.size() * 4) != 0) {
            std::fprintf(stderr, "fufft::ref::fufft_pipeline_v16_bfp differs from the C call\n");
            return 44;
         }
         refs++;
      }
      // run_large<N, LOUT, ROUT, MID, MLEAD, MNRV>: the reference bench's own
      // configuration, one chained filter per transform; a split the library
      // does not run is refused before any launch
      {
         const int64_t nl = 32768, bl = 2;
         std::vector<float> tl(2 * nl * bl), fl2(2 * nl * bl), xl(2 * nl * bl), a1(2 * nl * bl), a2(2 * nl * bl);
         for(auto& v : tl) v = rng.next();
         for(auto& v : xl) v = rng.next();
         for(int64_t t = 0; t < bl; t++)
            CHECK_FU(fufft_plan_filter_large_f32(nl, FUFFT_V16, FUFFT_FILTER_TAPS, 1, tl.data() + 2 * t * nl,
                                                 fl2.data() + 2 * t * nl));
         void* d_l = nullptr; void* d_lf = nullptr;
         CHECK_HIP(hipMalloc(&d_l, (size_t)nl * bl * 8)); CHECK_HIP(hipMalloc(&d_lf, (size_t)nl * bl * 8));
         CHECK_HIP(hipMemcpy(d_lf, fl2.data(), (size_t)nl * bl * 8, hipMemcpyHostToDevice));
         CHECK_HIP(hipMemcpy(d_l, xl.data(), (size_t)nl * bl * 8, hipMemcpyHostToDevice));
         CHECK_FU(fufft_conv_large_f32(d_l, d_lf, nl, nl, bl, FUFFT_MID_MUL, FUFFT_V16, s));
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(a1.data(), d_l, (size_t)nl * bl * 8, hipMemcpyDeviceToHost));
         CHECK_HIP(hipMemcpy(d_l, xl.data(), (size_t)nl * bl * 8, hipMemcpyHostToDevice));
         CHECK_FU((fufft::ref::run_large<32768, 1, 16, 2048, 8, 2>(d_l, d_lf, bl, s)));
         CHECK_HIP(hipStreamSynchronize(s));
         CHECK_HIP(hipMemcpy(a2.data(), d_l, (size_t)nl * bl * 8, hipMemcpyDeviceToHost));
         const int refused = fufft::ref::run_large<32768, 2, 16, 128, 8, 1>(d_l, d_lf, bl, s);
         CHECK_HIP(hipFree(d_l)); CHECK_HIP(hipFree(d_lf));
         if(!same_bits(a1, a2)) { std::fprintf(stderr, "fufft::ref::run_large differs from the C call\n"); return 45; }
         if(refused != FUFFT_ERR_UNSUPPORTED) { std::fprintf(stderr, "run_large ran a split the library does not\n"); return 46; }
         refs++;
      }
      CHECK_HIP(hipFree(d_f16)); CHECK_HIP(hipFree(d_f8)); CHECK_HIP(hipFree(d_fbp));
   }

   CHECK_HIP(hipFree(d_a)); CHECK_HIP(hipFree(d_f)); CHECK_HIP(hipFree(d_o));
   CHECK_HIP(hipFree(d_o2)); CHECK_HIP(hipFree(d_spec));
   CHECK_HIP(hipStreamDestroy(s));
   std::printf("ok C++ caller: n=%lld batch=%lld, template == C entry == split == in place, rel L2 vs fp64 direct %.2e; "
               "reference-format BFP == its definition; 64x64 2D rel L2 %.2e; %d plan objects == their C calls; "
               "%d reference-named launches == their C calls\n",
               (long long)n, (long long)batch, rel, rel2, plans, refs);
   return 0;
}
