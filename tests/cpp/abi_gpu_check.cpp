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
//     cyclic convolution, rel L2 <= 2e-6.
// Built by fufft_amd/build.py into tests/cpp/_build/abi_gpu_check and run by
// tests/test_gpu_cpp_caller.py.  Prints "ok ..." and returns 0 on success.
#include "fufft/fufft.hpp"

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

   CHECK_HIP(hipFree(d_a)); CHECK_HIP(hipFree(d_f)); CHECK_HIP(hipFree(d_o));
   CHECK_HIP(hipFree(d_o2)); CHECK_HIP(hipFree(d_spec));
   CHECK_HIP(hipStreamDestroy(s));
   std::printf("ok C++ caller: n=%lld batch=%lld, template == C entry == split == in place, rel L2 vs fp64 direct %.2e; "
               "reference-format BFP == its definition; 64x64 2D rel L2 %.2e\n",
               (long long)n, (long long)batch, rel, rel2);
   return 0;
}
