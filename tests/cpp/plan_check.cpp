// Host-side checks of include/fufft/plan.hpp (no GPU needed): the header
// compiles, and every plan object rejects bad arguments with fufft::Error
// carrying the C ABI status before it allocates or touches the device.
// Built and run by tests/test_library_cpu.py.  Prints "ok" and returns 0.
#include "fufft/plan.hpp"

#include <cstdio>
#include <vector>

namespace {

template<class F>
int status_of(F&& f)
{
   try {
      f();
   } catch(const fufft::Error& e) {
      return e.status();
   }
   return FUFFT_OK;
}

}  // namespace

int main()
{
   std::vector<float> taps(2 * 65536, 0.5f);
   // unsupported sizes: the fastest-variant lookup, the four-step plan and the 2D planner refuse them
   if(status_of([&] { fufft::Conv1d<> c(1000, taps.data()); }) != FUFFT_ERR_UNSUPPORTED) return 1;
   if(status_of([&] { fufft::ConvLarge<> c(4096, taps.data()); }) != FUFFT_ERR_UNSUPPORTED) return 2;
   if(status_of([&] { fufft::Conv2d<> c(512, 100, taps.data()); }) != FUFFT_ERR_UNSUPPORTED) return 3;
   // missing filter data, a zero filter count, an unknown layout or kind
   if(status_of([&] { fufft::Conv1d<> c(4096, nullptr); }) != FUFFT_ERR_INVALID) return 4;
   if(status_of([&] { fufft::Conv1d<> c(4096, taps.data(), 0); }) != FUFFT_ERR_INVALID) return 5;
   if(status_of([&] { fufft::Conv1d<> c(4096, taps.data(), 1, FUFFT_FILTER_TAPS, 9); }) != FUFFT_ERR_INVALID) return 6;
   if(status_of([&] { fufft::Conv1d<> c(4096, taps.data(), 1, 7, FUFFT_LAYOUT_DR, fufft::Variant::V16); }) !=
      FUFFT_ERR_INVALID)
      return 7;
   if(status_of([&] { fufft::ConvBfpScaled<> c(4096, nullptr); }) != FUFFT_ERR_INVALID) return 8;
   if(status_of([&] { fufft::ConvLarge<> c(32768, taps.data(), 1, FUFFT_FILTER_TAPS, fufft::Variant(7)); }) !=
      FUFFT_ERR_INVALID)
      return 9;
   if(status_of([&] { fufft::Conv2d<> c(512, 512, taps.data(), 1, FUFFT_FILTER_TAPS, 7); }) != FUFFT_ERR_INVALID)
      return 10;
   // an Error names where it came from
   try {
      fufft::Conv1d<> c(1000, taps.data());
   } catch(const fufft::Error& e) {
      if(std::string(e.what()).find("fufft_fastest_variant") == std::string::npos) return 11;
   }
   std::printf("ok plan objects reject bad arguments before any device call\n");
   return 0;
}
