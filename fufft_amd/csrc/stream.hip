// HBM stream ceiling for gfx950: a device copy made of the same buffer
// instructions the conv kernels use, as the measured bandwidth the conv
// kernels are compared with, and as the copy of known size that scales the
// rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes.
//
// A workgroup of 256 lanes copies one tile of kTile bytes: kUnroll 16-byte
// loads per lane, each wavefront instruction a contiguous KiB, all in flight
// before the stores.  The tile's base goes into a wave-uniform buffer
// resource whose size is the bytes left from that base, so the hardware's
// range check (loads beyond it return 0, stores beyond it are dropped) covers
// a last, partial tile.  nontemporal adds the streaming cache policy (NT) to
// the loads and stores.
#include "fufft_device.hpp"
#include "fufft_internal.hpp"

namespace fufft {

namespace {

constexpr int      kLanes  = 256;
constexpr int      kUnroll = 8;
constexpr uint64_t kTile   = (uint64_t)kLanes * 16 * kUnroll;   // 32 KiB
// cache-policy bits of the buffer instructions on gfx950: NT (bit 1)
constexpr int      kNT     = 2;

template<int POLICY>
__global__ void __launch_bounds__(kLanes) stream_kernel(const char* in, char* out, uint64_t bytes)
{
   typedef uint32_t u4 __attribute__((ext_vector_type(4)));
   const uint64_t base = (uint64_t)blockIdx.x * kTile;
   const uint64_t left = bytes - base;
   const uint32_t size = left < kTile ? (uint32_t)left : (uint32_t)kTile;
   const __amdgpu_buffer_rsrc_t ri =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(in) + base, 0, (int)size, Buf::kFlags);
   const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(out + base, 0, (int)size, Buf::kFlags);
   const uint32_t off = threadIdx.x * 16u;
   u4 v[kUnroll];
#pragma unroll
   for(int u = 0; u < kUnroll; u++)
      v[u] = __builtin_amdgcn_raw_buffer_load_b128(ri, off, u * kLanes * 16, POLICY);
#pragma unroll
   for(int u = 0; u < kUnroll; u++)
      __builtin_amdgcn_raw_buffer_store_b128(v[u], ro, off, u * kLanes * 16, POLICY);
}

}  // namespace

hipError_t launch_stream(const void* in, void* out, uint64_t bytes, bool nontemporal, hipStream_t s)
{
   if(bytes == 0) return hipSuccess;
   const uint64_t tiles = (bytes + kTile - 1) / kTile;
   if(tiles > 0x7fffffffull) return hipErrorInvalidValue;
   const void* k = nontemporal ? reinterpret_cast<const void*>(&stream_kernel<kNT>)
                               : reinterpret_cast<const void*>(&stream_kernel<0>);
   const char* pi = static_cast<const char*>(in);
   char* po = static_cast<char*>(out);
   uint64_t b = bytes;
   void* argv[] = { &pi, &po, &b };
   return hipLaunchKernel(k, dim3((unsigned)tiles), dim3(kLanes), argv, 0, s);
}

}  // namespace fufft
