// extern "C" entry points over the reference's fp64 mixed-radix CPU conv path
// (cpu_mixed.cpp), compiled where it lies (included by path through
// -I$(REF)); nothing from it is copied into this repository.  This is the CPU
// path bench.py times as its "reference" CPU baseline.
#include "cpu_mixed.cpp"

#include <cstdint>

extern "C" {

int ref_mixed_main(void) { return fufft_ref_mixed_main(); }

int ref_mixed_factorise(int N, int V, int* R) { return factorise(N, V, R); }
int ref_mixed_mixedrev(int idx, const int* R, int p) { return mixedrev(idx, R, p); }

// cpu_mixed.cpp:260-266: fft_dif -> multiply by the digit-ordered spectrum ->
// fft_dit, per signal; complex arrays are interleaved double (re, im)
void ref_mixed_conv_f64(int N, int V, const double* a, const double* spec_dr,
                        int64_t spec_stride, double* out, int64_t batch)
{
   int R[16];
   const int p = factorise(N, V, R);
   for(int64_t t = 0; t < batch; t++) {
      cd* A = reinterpret_cast<cd*>(out) + t * N;
      const cd* x = reinterpret_cast<const cd*>(a) + t * N;
      const cd* s = reinterpret_cast<const cd*>(spec_dr) + t * spec_stride;
      for(int i = 0; i < N; i++) A[i] = x[i];
      fft_dif(A, N, -1, R, p, V);
      for(int i = 0; i < N; i++) A[i] *= s[i];
      fft_dit(A, N, +1, R, p, V);
   }
}

}  // extern "C"
