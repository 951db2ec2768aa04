// A C++ caller of the library on the GPU, with no Python anywhere: the HIP
// runtime for memory and streams, include/fufft/fufft.hpp for the calls.
// It convolves a seeded batch at N = 4096 (FUFFT_AUTO) three ways and checks:
//   - fufft::pipeline<MidMultiply> against an fp64 direct cyclic convolution
//     (O(N^2) per checked signal), rel L2 <= 2e-6;
//   - the raw C entry point fufft_conv_f32 bit for bit against the template;
//   - in place (in == out) bit for bit against out of place;
//   - the split path (pipeline_fwd + pipeline_apply) bit for bit against fused.
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

   CHECK_HIP(hipFree(d_a)); CHECK_HIP(hipFree(d_f)); CHECK_HIP(hipFree(d_o));
   CHECK_HIP(hipFree(d_o2)); CHECK_HIP(hipFree(d_spec));
   CHECK_HIP(hipStreamDestroy(s));
   std::printf("ok C++ caller: n=%lld batch=%lld, template == C entry == split == in place, rel L2 vs fp64 direct %.2e\n",
               (long long)n, (long long)batch, rel);
   return 0;
}
