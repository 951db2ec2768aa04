// Filter planning on the GPU: the digit-order gather of natural-order spectra.
//
// The reference plans filters on the host: the digit-order permutation and the
// 1/N fold (mixedrev_host, bench_fufft.cu:63-82, 156-170), the four-step chain
// order (bench_fufft.cu:410-428) and the 2D order (verify_kernel.cpp:738-748).
// This kernel does the permutation for spectra already in device memory:
// output position (r, c) of an h x w item (h = 1 in 1D) receives bin
// (rev_h(r), rev_w(c')) times scale, each rev a bit-group reversal over the
// plan's radix widths in pass order, c' = c or, lane-major, the digit-order
// slot that position c holds (lane_slot).  One thread per output point, so the
// writes are coalesced and the reads gather; planning runs once per filter,
// not on the conv's hot path.  (Taps are planned by the conv kernels' own
// forward half, K_PLAN_TAPS.)
#include "fufft_device.hpp"
#include "fufft_internal.hpp"

namespace fufft {

// digit 0 (the first pass's radix) is the most significant bit group of idx
// and becomes the least significant group of the result
__device__ __forceinline__ uint32_t group_reverse_dev(uint32_t idx, const GatherDigits& d)
{
   uint32_t out = 0;
   int pos = d.bits, op = 0;
   for(int i = 0; i < d.np; i++) {
      pos -= d.w[i];
      out |= ((idx >> pos) & ((1u << d.w[i]) - 1u)) << op;
      op += d.w[i];
   }
   return out;
}

__global__ void __launch_bounds__(256) gather_kernel(const GatherParams p)
{
   const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
   if(i >= p.total) return;
   const uint32_t lb = p.dh.bits + p.dw.bits;                 // log2 of the points per item
   const uint32_t per = 1u << lb;
   const uint64_t item = i >> lb;
   const uint32_t o = (uint32_t)(i & (per - 1u));
   const uint32_t r = o >> p.dw.bits;
   uint32_t c = o & ((1u << p.dw.bits) - 1u);
   if(p.lane_v) {
      // lane-major along the row (1D filters, 2D columns): the digit-order
      // slot that position c holds -- pairs, or the reference's bperm
      const uint32_t vlog = 31u - (uint32_t)__builtin_clz((uint32_t)p.lane_v);
      const uint32_t tlog = p.dw.bits - vlog;
      c = p.bperm ? ((c & ((1u << tlog) - 1u)) << vlog) | (c >> tlog) : lane_slot(c, tlog, vlog);
   }
   const uint32_t src = (group_reverse_dev(r, p.dh) << p.dw.bits) | group_reverse_dev(c, p.dw);
   const float2 v = p.in[item * per + src];
   p.out[i] = make_float2(v.x * p.scale, v.y * p.scale);
}

hipError_t launch_gather(const GatherParams& p, hipStream_t s)
{
   if(p.total == 0) return hipSuccess;
   if(p.dh.bits + p.dw.bits > 30 || p.dh.np > 32 || p.dw.np > 32) return hipErrorInvalidValue;
   const uint64_t blocks = (p.total + 255) / 256;
   if(blocks > 0x7fffffffull) return hipErrorInvalidValue;
   GatherParams arg = p;
   void* argv[] = { &arg };
   return hipLaunchKernel(reinterpret_cast<const void*>(&gather_kernel), dim3((unsigned)blocks),
                          dim3(256), argv, 0, s);
}

}  // namespace fufft
