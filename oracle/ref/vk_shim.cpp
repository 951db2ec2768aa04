// extern "C" entry points over the reference's own CPU transcription of its
// device code (verify_kernel.cpp).  The reference source is compiled where it
// lies -- this file includes it by path through -I$(REF) -- and nothing from it
// is copied into this repository.  The built library lands in oracle/_ref/ and
// is used only by tests/ (to pin the oracle) and by bench.py's CPU baseline.
//
// Complex arrays are interleaved float (re, im), which is the layout of
// std::complex<float>.  Filters are per signal (n = N * batch entries), as the
// reference's kernels index them (verify_kernel.cpp:229, 1077).
#include "verify_kernel.cpp"

#include <algorithm>
#include <cstdint>

namespace {
std::vector<cf> vec(const float* p, size_t n)
{
   const cf* c = reinterpret_cast<const cf*>(p);
   return std::vector<cf>(c, c + n);
}
void put(const std::vector<cf>& v, float* p)
{
   std::copy(v.begin(), v.end(), reinterpret_cast<cf*>(p));
}
}

extern "C" {

int ref_vk_main(void) { return fufft_ref_vk_main(); }

int ref_vk_mixedrev(int idx, int lead, int nr8) { return mixedrev(idx, lead, nr8); }
int ref_vk_mixedrev16(int idx, int lead, int nr16) { return mixedrev16(idx, lead, nr16); }
int ref_vk_chain_rev(int idx, const int* radices, int np)
{
   return chain_rev(idx, std::vector<int>(radices, radices + np));
}

// verify_kernel.cpp:1051-1082 (fufft_pipeline_v16)
void ref_vk_pipeline_v16(int N, int lead, int nrv, int cpb, const float* a,
                         const float* bspec, float* out, int batch)
{
   const size_t n = (size_t)N * batch;
   std::vector<cf> o;
   kernel_pipeline_v16(N, lead, nrv, cpb, CPP_OPT, vec(a, n), vec(bspec, n), o, batch);
   put(o, out);
}

// verify_kernel.cpp:1012-1049 (fufft_pipeline_v16f, lane-major filter)
void ref_vk_pipeline_v16f(int N, int lead, int nrv, int cpb, const float* a,
                          const float* bperm, float* out, int batch)
{
   const size_t n = (size_t)N * batch;
   std::vector<cf> o;
   kernel_pipeline_v16f(N, lead, nrv, cpb, CPP_OPT, vec(a, n), vec(bperm, n), o, batch);
   put(o, out);
}

// verify_kernel.cpp:1183-1203 (fufft_c2c: forward radix-8 Stockham, N = 8^k)
void ref_vk_c2c(int N, int cpb, const float* a, float* out, int batch)
{
   const size_t n = (size_t)N * batch;
   std::vector<cf> o;
   kernel_c2c(N, ilog8(N), cpb, CPP_OPT, vec(a, n), o, batch);
   put(o, out);
}

// verify_kernel.cpp:211-244 (fufft_pipeline_ip with MidMultiply)
void ref_vk_pipeline_ip(int N, int lead, int nr8, int cpb, const float* a,
                        const float* b_dr, float* out, int batch)
{
   const size_t n = (size_t)N * batch;
   std::vector<cf> o;
   kernel_pipeline_ip(N, lead, nr8, cpb, CPP_OPT, vec(a, n), vec(b_dr, n), o, batch);
   put(o, out);
}

// verify_kernel.cpp:794-836 (fufft_pipeline_fwd / fufft_pipeline_apply)
void ref_vk_pipeline_fwd(int N, int lead, int nr8, int cpb, const float* a,
                         float* spec, int batch)
{
   const size_t n = (size_t)N * batch;
   std::vector<cf> s;
   kernel_pipeline_fwd(N, lead, nr8, cpb, CPP_OPT, vec(a, n), s, batch);
   put(s, spec);
}

void ref_vk_pipeline_apply(int N, int lead, int nr8, int cpb, const float* spec,
                           const float* b_dr, float* out, int batch)
{
   const size_t n = (size_t)N * batch;
   std::vector<cf> o;
   kernel_pipeline_apply(N, lead, nr8, cpb, CPP_OPT, vec(spec, n), vec(b_dr, n), o, batch);
   put(o, out);
}

// verify_kernel.cpp:378-432 (four-step chain and its monolithic equivalent);
// A is transformed in place
void ref_vk_conv_foursteps_cfg(float* A, const float* b_dr, int N, int batch,
                               int r_out, int mid, int v16_mid)
{
   const size_t n = (size_t)N * batch;
   std::vector<cf> v = vec(A, n);
   conv_foursteps_cfg(v, vec(b_dr, n), N, batch, CPP_OPT, r_out, mid, v16_mid != 0);
   put(v, A);
}

void ref_vk_conv_monolithic_cfg(float* A, const float* b_dr, int N, int batch,
                                int r_out, int mid, int v16_mid)
{
   const size_t n = (size_t)N * batch;
   std::vector<cf> v = vec(A, n);
   conv_monolithic_cfg(v, vec(b_dr, n), N, batch, CPP_OPT, r_out, mid, v16_mid != 0);
   put(v, A);
}

// verify_kernel.cpp:700-722 (fufft_conv2d)
void ref_vk_conv2d(int H, int W, const float* a, const float* b_dr, float* out, int batch)
{
   const size_t n = (size_t)H * W * batch;
   std::vector<cf> o;
   kernel_conv2d(H, W, CPP_OPT, vec(a, n), vec(b_dr, n), o, batch);
   put(o, out);
}

// verify_kernel.cpp:580-615 (fufft_conv_r2)
void ref_vk_conv_r2(int N, int lead, int nr8, int cpb, const float* xr, const float* yr,
                    const float* b_dr, float* ur, float* vr, int batch)
{
   const size_t n = (size_t)N * batch;
   std::vector<float> x(xr, xr + n), y(yr, yr + n), u, v;
   kernel_conv_r2(N, lead, nr8, cpb, CPP_OPT, x, y, vec(b_dr, n), u, v, batch);
   std::copy(u.begin(), u.end(), ur);
   std::copy(v.begin(), v.end(), vr);
}

// verify_kernel.cpp:1092-1135 (per-transform fp32-scale BFP, for reference)
float ref_vk_bfp_quantize(const float* x, int N, int16_t* q)
{
   BfpQuant b = bfp_quantize(reinterpret_cast<const cf*>(x), N);
   for(int i = 0; i < N; i++) { q[2 * i] = b.qre[i]; q[2 * i + 1] = b.qim[i]; }
   return b.scale;
}

// verify_kernel.cpp:1111-1135 (kernel_v16_bfp, the fufft_pipeline_v16_bfp
// dataflow): batch transforms of N points, each input as int16 pairs with its
// own fp32 scale, one shared filter (int16 pairs, one scale); writes the
// output pairs and scales
void ref_vk_v16_bfp(int N, int lead, int nrv, const int16_t* aq, const float* ascale,
                    const int16_t* bq, float bscale, int16_t* oq, float* oscale, int batch)
{
   BfpQuant a, b, o;
   a.qre.resize(N); a.qim.resize(N); b.qre.resize(N); b.qim.resize(N);
   for(int i = 0; i < N; i++) { b.qre[i] = bq[2 * i]; b.qim[i] = bq[2 * i + 1]; }
   b.scale = bscale;
   for(int t = 0; t < batch; t++) {
      const int16_t* at = aq + (size_t)2 * N * t;
      for(int i = 0; i < N; i++) { a.qre[i] = at[2 * i]; a.qim[i] = at[2 * i + 1]; }
      a.scale = ascale[t];
      kernel_v16_bfp(N, lead, nrv, CPP_OPT, a, b, o);
      int16_t* ot = oq + (size_t)2 * N * t;
      for(int i = 0; i < N; i++) { ot[2 * i] = o.qre[i]; ot[2 * i + 1] = o.qim[i]; }
      oscale[t] = o.scale;
   }
}

}  // extern "C"
