// 1D fused cyclic convolution for gfx950: forward DIF -> mid operation ->
// inverse DIT in one launch, plus the split forward / apply kernels and the
// two-for-one real variant.
//
// Replaces the reference kernels fufft_pipeline_v16 / _v16f / _wide
// (fufft.cuh:1499-1534, 1703-1734), fufft_pipeline_ip / _fused
// (fufft.cuh:1757-1791), fufft_pipeline_fwd / _apply (fufft.cuh:1343-1407) and
// fufft_conv_r2 (fufft.cuh:1273-1330).
//
// Mapping to CDNA4.  A transform of N points is held by T = N/V lanes with V
// values each (V = 16: radix-16 passes; V = 8: radix-8 passes).  T <= 64
// packs 64/T transforms into one wavefront and needs no workgroup barrier at
// all; T > 64 gives one transform per workgroup of T/64 wavefronts.  HBM is
// touched exactly three times per point: the first DIF pass reads the signal
// straight into registers, the mid operation reads the filter in registers at
// the M = 1 boundary, and the last DIT pass writes the result straight from
// registers.  Every other pass boundary is an exchange through LDS.
#include "fufft_device.hpp"
#include "fufft_plan.hpp"
#include "fufft_internal.hpp"

namespace fufft {

constexpr int cpb_for(int T) { return T >= 128 ? 1 : 256 / T; }

template<int N, int V, int LAYOUT, int KIND>
__global__ void __launch_bounds__(cpb_for(N / V) * (N / V))
conv1d_kernel(const Conv1dParams p)
{
   using PL = Plan<N, V>;
   using LD = Lds<V, LAYOUT>;
   constexpr int T     = PL::T;
   constexpr int CPB   = cpb_for(T);
   constexpr int SLOT  = LD::size(N);
   constexpr int LANES = T < 64 ? 64 : T;

   extern __shared__ float2 lds[];
   const int slot = threadIdx.x / T;
   const int L    = threadIdx.x % T;
   const uint32_t t = blockIdx.x * CPB + slot;
   if(t >= p.ntrans) return;                 // T > 64 => CPB == 1: whole group leaves

   float2* A = lds + slot * SLOT;
   const size_t base = (size_t)t * N;
   Twiddles<PL> tw;
   tw.load(p.tw, L);
   float2 r[V];

   if constexpr(KIND == K_APPLY) {
      // spectrum positions L*V .. L*V+V-1, two complex per 16-byte load
      const float4* s = reinterpret_cast<const float4*>(
         static_cast<const float2*>(p.spec) + (size_t)(t % p.scount) * N + L * V);
#pragma unroll
      for(int m = 0; m < V / 2; m++) {
         const float4 q = s[m];
         r[2 * m] = make_float2(q.x, q.y);
         r[2 * m + 1] = make_float2(q.z, q.w);
      }
   } else {
      if constexpr(KIND == K_CONV_R2) {
         const float* x = static_cast<const float*>(p.in0) + base;
         const float* y = static_cast<const float*>(p.in1) + base;
#pragma unroll
         for(int q = 0; q < V; q++) r[q] = make_float2(x[L + q * T], y[L + q * T]);
      } else {
         const float2* x = static_cast<const float2*>(p.in0) + base;
#pragma unroll
         for(int q = 0; q < V; q++) r[q] = x[L + q * T];
      }
      forward_dif<PL, LD, LANES>(r, A, L, tw);
   }

   if constexpr(KIND == K_FWD) {
      float4* s = reinterpret_cast<float4*>(static_cast<float2*>(p.out0) + base + L * V);
#pragma unroll
      for(int m = 0; m < V / 2; m++)
         s[m] = make_float4(r[2 * m].x, r[2 * m].y, r[2 * m + 1].x, r[2 * m + 1].y);
      return;
   } else {
      mid_op<PL>(r, static_cast<const float2*>(p.filt) + (size_t)(t % p.fcount) * N, L, p.mid, p.fl);
      inverse_dit<PL, LD, LANES>(r, A, L, tw);

      if constexpr(KIND == K_CONV_R2) {
         float* u = static_cast<float*>(p.out0) + base;
         float* v = static_cast<float*>(p.out1) + base;
#pragma unroll
         for(int q = 0; q < V; q++) { u[L + q * T] = r[q].x; v[L + q * T] = r[q].y; }
      } else {
         float2* o = static_cast<float2*>(p.out0) + base;
#pragma unroll
         for(int q = 0; q < V; q++) o[L + q * T] = r[q];
      }
   }
}

template<int N, int V, int LAYOUT, int KIND>
static hipError_t launch_one(const Conv1dParams& p, hipStream_t s)
{
   constexpr int T = N / V, CPB = cpb_for(T);
   const size_t shm = (size_t)CPB * Lds<V, LAYOUT>::size(N) * sizeof(float2);
   const void* k = reinterpret_cast<const void*>(&conv1d_kernel<N, V, LAYOUT, KIND>);
   if(shm > 65536) {
      const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
      if(e != hipSuccess) return e;
   }
   const dim3 grid((p.ntrans + CPB - 1) / CPB), block(CPB * T);
   Conv1dParams arg = p;
   void* argv[] = { &arg };
   return hipLaunchKernel(k, grid, block, argv, shm, s);
}

template<int N, int V, int LAYOUT>
static hipError_t launch_kind(int kind, const Conv1dParams& p, hipStream_t s)
{
   switch(kind) {
      case K_CONV:    return launch_one<N, V, LAYOUT, K_CONV>(p, s);
      case K_CONV_R2: return launch_one<N, V, LAYOUT, K_CONV_R2>(p, s);
      case K_FWD:     return launch_one<N, V, LAYOUT, K_FWD>(p, s);
      case K_APPLY:   return launch_one<N, V, LAYOUT, K_APPLY>(p, s);
      default:        return hipErrorInvalidValue;
   }
}

template<int N, int V>
static hipError_t launch_nv(int kind, int layout, const Conv1dParams& p, hipStream_t s)
{
   return layout == LAYOUT_PAD ? launch_kind<N, V, LAYOUT_PAD>(kind, p, s)
                               : launch_kind<N, V, LAYOUT_XOR>(kind, p, s);
}

bool conv1d_supported(int n, int v)
{
   if(v == 16) return n >= 256 && n <= 16384 && (n & (n - 1)) == 0;
   if(v == 8)  return n >= 512 && n <= 4096 && (n & (n - 1)) == 0;
   return false;
}

hipError_t launch_conv1d(int kind, int n, int v, int layout, const Conv1dParams& p, hipStream_t s)
{
   if(v == 16) {
      switch(n) {
         case 256:   return launch_nv<256, 16>(kind, layout, p, s);
         case 512:   return launch_nv<512, 16>(kind, layout, p, s);
         case 1024:  return launch_nv<1024, 16>(kind, layout, p, s);
         case 2048:  return launch_nv<2048, 16>(kind, layout, p, s);
         case 4096:  return launch_nv<4096, 16>(kind, layout, p, s);
         case 8192:  return launch_nv<8192, 16>(kind, layout, p, s);
         case 16384: return launch_nv<16384, 16>(kind, layout, p, s);
         default:    break;
      }
   } else if(v == 8) {
      switch(n) {
         case 512:  return launch_nv<512, 8>(kind, layout, p, s);
         case 1024: return launch_nv<1024, 8>(kind, layout, p, s);
         case 2048: return launch_nv<2048, 8>(kind, layout, p, s);
         case 4096: return launch_nv<4096, 8>(kind, layout, p, s);
         default:   break;
      }
   }
   return hipErrorInvalidValue;
}

}  // namespace fufft
