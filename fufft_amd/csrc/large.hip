// Four-step large-N outer levels for gfx950.
//
// Replaces fufft_outer_pass_r<16, SIGN, DIT> (fufft.cuh:1113-1140): one flat
// radix-16 level of the in-place DIF (forward) or DIT (inverse) chain, over a
// batch of n-point transforms in HBM.  Thread = one butterfly group (b, j) of
// a level with stride M: taps b*16*M + j + k*M, k = 0..15.  Consecutive
// threads take consecutive j, so every tap load of a wavefront is one
// contiguous 512-byte run.  Stage twiddles W_{16M}^(jk) come from the base
// W^j in the table and the single multiplicative chain, in the same
// operation order as the in-workgroup passes, so the whole four-step chain is
// bit-identical to the monolithic chain with the outer radix-16 levels first.
#include "fufft_device.hpp"
#include "fufft_internal.hpp"

namespace fufft {

struct OuterParams {
   float2*       buf;
   const float2* tw;
   uint32_t      n;         // transform length
   uint32_t      log_gpt;   // log2(n / 16): groups per transform
   uint32_t      log_m;     // log2(M)
   uint32_t      groups;    // groups in the launch (batch * n / 16)
};

template<int SIGN, bool DIT>
__global__ void __launch_bounds__(256) outer_pass_kernel(const OuterParams p)
{
   const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
   if(gid >= p.groups) return;
   // n / 16 >= 512 groups per transform, so a wavefront never straddles two
   // transforms and the transform index is uniform
   const uint32_t t  = (uint32_t)uniform((int)(gid >> p.log_gpt));
   const uint32_t gi = gid & ((1u << p.log_gpt) - 1u);
   const uint32_t M  = 1u << p.log_m;
   const uint32_t j  = gi & (M - 1u);
   const uint32_t b  = gi >> p.log_m;

   const Buf io(p.buf + (size_t)t * p.n, p.n * 8u);
   const uint32_t voff = ((b << (p.log_m + 4)) + j) * 8u;
   const uint32_t kst  = M * 8u;

   float2 r[16];
#pragma unroll
   for(int k = 0; k < 16; k++) r[k] = io.ld2(voff, k * kst);

   const Buf tb(p.tw, FUFFT_TW_ENTRIES * 8u);
   const float2 base = tb.ld2(j * 8u, 16u * M * 8u);            // W_{16M}^j
   const float2 w1 = SIGN < 0 ? make_float2(base.x, -base.y) : base;
   if constexpr(DIT) twiddle_group<16, CHAIN_SINGLE, 0, 1>(r, w1);
   dftR<16, SIGN, 0, 1>(r);
   if constexpr(!DIT) twiddle_group<16, CHAIN_SINGLE, 0, 1>(r, w1);

#pragma unroll
   for(int k = 0; k < 16; k++) io.st2(r[k], voff, k * kst);
}

hipError_t launch_outer_pass(float2* buf, int64_t n, int64_t batch, int64_t M, bool dit,
                             const float2* tw, hipStream_t s)
{
   int log_n = 0, log_m = 0;
   while(((int64_t)1 << log_n) < n) log_n++;
   while(((int64_t)1 << log_m) < M) log_m++;
   const int64_t groups = batch * (n / 16);
   if(n < 8192 || n > ((int64_t)1 << FUFFT_TW_LOG_MAX) || 16 * M > n || groups > 0xffffffffll)
      return hipErrorInvalidValue;
   OuterParams p{buf, tw, (uint32_t)n, (uint32_t)(log_n - 4), (uint32_t)log_m, (uint32_t)groups};
   const dim3 grid((unsigned)((groups + 255) / 256)), block(256);
   const void* k = dit ? reinterpret_cast<const void*>(&outer_pass_kernel<+1, true>)
                       : reinterpret_cast<const void*>(&outer_pass_kernel<-1, false>);
   void* argv[] = { &p };
   return hipLaunchKernel(k, grid, block, argv, 0, s);
}

}  // namespace fufft
