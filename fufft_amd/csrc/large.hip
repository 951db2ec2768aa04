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

// ---- two outer levels in one pass ----------------------------------------------------
// With two outer levels (n = 16 * 16 * mid, strides M1 = n/16 and M2 = n/256)
// the 256 points j + k1*M1 + k2*M2 (k1, k2 < 16) of one j < M2 are closed under
// both levels: the level-M1 groups are j1 = j + k2*M2 (taps over k1), the
// level-M2 groups are (b = k1, j) (taps over k2).  A workgroup takes 16
// consecutive j of one transform (4096 points, 32 KiB through LDS): the first
// level runs in registers straight from HBM, the second after one exchange,
// and the result goes back to HBM -- one read and one write of the data for
// the two levels instead of two of each.  Every group runs exactly the
// butterfly and twiddle chain of outer_pass_kernel, so results are bit-identical
// to two launches of it.  Forward (DIF): level M1 then M2; inverse (DIT): M2
// then M1.
struct Outer2Params {
   float2*       buf;
   const float2* tw;
   uint32_t      n;
   uint32_t      log_m2;    // log2(n / 256)
   uint32_t      tiles;     // 16-wide tiles of j per transform: n / 4096
   uint32_t      ntiles;    // tiles in the launch
};

// LDS slot of (k1, k2, jj): rows of 16 jj, k2 rows per k1 block, k1 blocks of
// 256 + 16 so that the two k1 rows of a half-wavefront land 16 banks apart
constexpr int kOuter2Row = 16 * 16 + 16;
__device__ __forceinline__ int outer2_slot(int k1, int k2, int jj) { return k1 * kOuter2Row + k2 * 16 + jj; }

template<int SIGN>
__device__ __forceinline__ void outer_group(float2 (&r)[16], const Buf& tb, uint32_t j, uint32_t M, bool dit)
{
   const float2 base = tb.ld2(j * 8u, 16u * M * 8u);              // W_{16M}^j
   const float2 w1 = SIGN < 0 ? make_float2(base.x, -base.y) : base;
   if(dit) twiddle_group<16, CHAIN_SINGLE, 0, 1>(r, w1);
   dftR<16, SIGN, 0, 1>(r);
   if(!dit) twiddle_group<16, CHAIN_SINGLE, 0, 1>(r, w1);
}

template<int SIGN, bool DIT>
__global__ void __launch_bounds__(256) outer2_kernel(const Outer2Params p)
{
   __shared__ float2 lds[16 * kOuter2Row];
   if(blockIdx.x >= p.ntiles) return;                             // whole workgroup
   const uint32_t t  = blockIdx.x / p.tiles;
   const uint32_t j0 = (blockIdx.x - t * p.tiles) * 16u;
   const int jj = threadIdx.x & 15;
   const int hi = threadIdx.x >> 4;                               // k2 in the first half, k1 in the second (DIF)
   const uint32_t M2 = 1u << p.log_m2, M1 = M2 << 4;
   const uint32_t j = j0 + (uint32_t)jj;

   const Buf io(p.buf + (size_t)t * p.n, p.n * 8u);
   const Buf tb(p.tw, FUFFT_TW_ENTRIES * 8u);
   float2 r[16];
   if constexpr(!DIT) {
      // level M1: group j1 = j + k2*M2, taps over k1
      const uint32_t k2 = (uint32_t)hi;
      const uint32_t voff = (j + k2 * M2) * 8u;
#pragma unroll
      for(int k1 = 0; k1 < 16; k1++) r[k1] = io.ld2(voff, k1 * M1 * 8u);
      outer_group<SIGN>(r, tb, j + k2 * M2, M1, false);
#pragma unroll
      for(int k1 = 0; k1 < 16; k1++) lds[outer2_slot(k1, (int)k2, jj)] = r[k1];
      __syncthreads();
      // level M2: group (b = k1, j), taps over k2
      const int k1 = hi;
#pragma unroll
      for(int q = 0; q < 16; q++) r[q] = lds[outer2_slot(k1, q, jj)];
      outer_group<SIGN>(r, tb, j, M2, false);
      const uint32_t vo2 = (j + (uint32_t)k1 * M1) * 8u;
#pragma unroll
      for(int q = 0; q < 16; q++) io.st2(r[q], vo2, q * M2 * 8u);
   } else {
      // level M2 first: group (b = k1, j), taps over k2
      const uint32_t k1 = (uint32_t)hi;
      const uint32_t voff = (j + k1 * M1) * 8u;
#pragma unroll
      for(int q = 0; q < 16; q++) r[q] = io.ld2(voff, q * M2 * 8u);
      outer_group<SIGN>(r, tb, j, M2, true);
#pragma unroll
      for(int q = 0; q < 16; q++) lds[outer2_slot((int)k1, q, jj)] = r[q];
      __syncthreads();
      // then level M1: group j1 = j + k2*M2, taps over k1
      const int k2 = hi;
#pragma unroll
      for(int q = 0; q < 16; q++) r[q] = lds[outer2_slot(q, k2, jj)];
      outer_group<SIGN>(r, tb, j + (uint32_t)k2 * M2, M1, true);
      const uint32_t vo2 = (j + (uint32_t)k2 * M2) * 8u;
#pragma unroll
      for(int q = 0; q < 16; q++) io.st2(r[q], vo2, q * M1 * 8u);
   }
}

hipError_t launch_outer2_pass(float2* buf, int64_t n, int64_t batch, bool dit, const float2* tw,
                              hipStream_t s)
{
   int log_n = 0;
   while(((int64_t)1 << log_n) < n) log_n++;
   if(((int64_t)1 << log_n) != n || n < (int64_t)1 << 17 || n > ((int64_t)1 << FUFFT_TW_LOG_MAX))
      return hipErrorInvalidValue;
   const int64_t tiles = n / 4096, ntiles = batch * tiles;
   if(ntiles > 0x7fffffffll) return hipErrorInvalidValue;
   Outer2Params p{buf, tw, (uint32_t)n, (uint32_t)(log_n - 8), (uint32_t)tiles, (uint32_t)ntiles};
   const void* k = dit ? reinterpret_cast<const void*>(&outer2_kernel<+1, true>)
                       : reinterpret_cast<const void*>(&outer2_kernel<-1, false>);
   void* argv[] = { &p };
   return hipLaunchKernel(k, dim3((unsigned)ntiles), dim3(256), argv, 0, s);
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
