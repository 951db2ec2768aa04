// Host-only check of the C++ mirror header: planning calls and status codes
// (no device work).  Built and run by tests/test_library_cpu.py.
#include "fufft/fufft.hpp"

#include <cstdio>

int main()
{
   const int64_t n = 4096;
   std::vector<float> taps(2 * n, 0.0f), filt(2 * n);
   taps[0] = 1.0f;                                  // delta taps: flat spectrum 1/n
   if(fufft::plan_filter(taps.data(), filt.data(), n) != FUFFT_OK) return 1;
   for(int64_t i = 0; i < n; i++)
      if(filt[2 * i] != 1.0f / n || filt[2 * i + 1] != 0.0f) return 2;
   const std::vector<int32_t> perm = fufft::digit_order(n);
   std::vector<int> seen(n, 0);
   for(int32_t p : perm) seen[p]++;
   for(int s : seen) if(s != 1) return 3;          // a permutation
   // argument errors come back before any device call
   if(fufft::pipeline<fufft::MidConjMultiply>(nullptr, nullptr, nullptr, n, 1) != FUFFT_ERR_INVALID) return 4;
   if(fufft::pipeline<fufft::MidMultiply>(nullptr, nullptr, nullptr, 1000, 1) != FUFFT_ERR_UNSUPPORTED) return 5;
   if(fufft::conv_large<fufft::MidNothing>(nullptr, nullptr, 1024, 1) != FUFFT_ERR_UNSUPPORTED) return 6;
   if(!fufft::supported(n) || fufft::supported(100)) return 7;
   if(!fufft::abi_matches()) return 18;
   {
      fufft::Variant a = fufft::Variant::Auto, b = fufft::Variant::Auto, c = fufft::Variant::Auto;
      if(fufft::fastest_variant(4096, &a) != FUFFT_OK || a != fufft::Variant::V16 ||
         fufft::fastest_variant(512, &b) != FUFFT_OK || b != fufft::Variant::R8 ||
         fufft::fastest_variant(4096, &c, FUFFT_LAYOUT_DR) != FUFFT_OK || c != fufft::Variant::R8) return 14;
      // an unsupported size or an unknown layout comes back as a status, the output untouched
      fufft::Variant d = fufft::Variant::Auto;
      if(fufft::fastest_variant(1000, &d) != FUFFT_ERR_UNSUPPORTED || d != fufft::Variant::Auto ||
         fufft::fastest_variant(4096, &d, 9) != FUFFT_ERR_INVALID || d != fufft::Variant::Auto) return 17;
   }
   if(!fufft::reads_filter<fufft::MidMultiply>() || !fufft::reads_filter<fufft::MidConjMultiply>() ||
      fufft::reads_filter<fufft::MidNothing>() || fufft::mid_reads_filter(3) != FUFFT_ERR_INVALID) return 15;
   if(fufft::c2c<FUFFT_INVERSE>(nullptr, nullptr, n, 1) != FUFFT_ERR_INVALID) return 8;
   if(fufft::pipeline_bfp_scaled(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, n, 1) != FUFFT_ERR_INVALID)
      return 16;
   if(fufft::plan_filter_device(nullptr, nullptr, n) != FUFFT_ERR_INVALID) return 9;
   if(fufft::pipeline_timed<fufft::MidMultiply>(nullptr, nullptr, nullptr, n, 1, nullptr, 0) != FUFFT_ERR_INVALID) return 10;
   if(fufft::plan_filter_large_device(nullptr, nullptr, 4096) != FUFFT_ERR_UNSUPPORTED) return 11;
   if(fufft::plan_filter2d_device(nullptr, nullptr, 512, 512) != FUFFT_ERR_INVALID) return 12;
   if(fufft_transforms_per_workgroup(4096, FUFFT_R8) != 1 || fufft_transforms_per_workgroup(512, FUFFT_R8) != 4) return 13;
   // the reference's launch surface by name: argument errors before any device
   // call, and a four-step split the library does not run refused as such
   {
      namespace R = fufft::ref;
      if((R::fufft_pipeline_v16<4096, 1, 3, 1>(nullptr, nullptr, fufft::MidMultiply{}, 1)) != FUFFT_ERR_INVALID) return 19;
      if((R::fufft_pipeline_ip<4096, 1, 4, 8, fufft::MidConjMultiply>(nullptr, nullptr, fufft::MidConjMultiply{}, 1)) !=
         FUFFT_ERR_INVALID) return 20;
      if((R::fufft_pipeline_v16_bfp<512, 2, 2, 16>(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1)) !=
         FUFFT_ERR_INVALID) return 21;
      if((R::fufft_c2c<512, 3, 1>(nullptr, nullptr, 1)) != FUFFT_ERR_INVALID) return 22;
      if((R::fufft_conv2d<64, 64, 1>(nullptr, nullptr, fufft::MidMultiply{}, 1)) != FUFFT_ERR_INVALID) return 23;
      if((R::run_large<32768, 1, 16, 2048, 8, 2>(nullptr, nullptr, 1)) != FUFFT_ERR_INVALID) return 24;
      if((R::run_large<32768, 2, 16, 128, 8, 1>(nullptr, nullptr, 1)) != FUFFT_ERR_UNSUPPORTED) return 25;
      if((R::run_large<65536, 1, 16, 4096, 1, 3>(nullptr, nullptr, 1)) != FUFFT_ERR_INVALID) return 26;
   }
   std::printf("ok %s\n", fufft::status_string(FUFFT_OK));
   return 0;
}
