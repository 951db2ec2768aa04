// HBM stream ceiling for gfx950: a device copy made of the same buffer
// instructions the conv kernels use, as the measured bandwidth the conv
// kernels are compared with, and as the copy of known size that scales the
// rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes.
//
// A workgroup of LANES lanes (64, 256 or 1024) copies tiles of
// LANES * W * LOADS bytes: LOADS loads of W bytes per lane (W = 16, or 8 as the
// conv kernels' float2 loads), each
// wavefront instruction one contiguous run of 64 * W bytes, all in flight
// before the stores.  Each tile's base goes into a wave-uniform buffer
// resource whose size is the bytes left from that base, so the hardware's
// range check (loads beyond it return 0, stores beyond it are dropped) covers
// a last, partial tile.
//
// The copy's shape is a parameter, so that the ceiling is the best of a sweep
// rather than one configuration:
//   - LANES: lanes per workgroup (64, 256, 1024);
//   - LOADS: loads in flight per lane (1 .. 32), W: bytes per load (8, 16);
//   - tiles per workgroup: consecutive tiles in a loop (per > 1), or a
//     persistent grid of `groups` workgroups striding over the tiles;
//   - the cache policy of the loads and of the stores, separately: the gfx950
//     buffer-instruction bits SC0 (1) and NT (2, streaming).
#include "fufft_device.hpp"
#include "fufft_internal.hpp"

#include <type_traits>

namespace fufft {

namespace {

// cache-policy bits of the buffer instructions on gfx950: SC0 (bit 0), NT (bit 1)
constexpr int kNT    = 2;


// Tile i of workgroup b: b * per + i (consecutive) or b + i * gridDim.x
// (grid-stride).  Every workgroup runs `per` iterations and leaves at the
// first tile past the end (a uniform branch), so every wave exits.
template<int LANES, int W, int LOADS, int PLD, int PST>
__global__ void __launch_bounds__(LANES)
stream_kernel(const char* in, char* out, uint64_t bytes, uint64_t tiles, uint32_t per, uint32_t stride)
{
   typedef uint32_t u4 __attribute__((ext_vector_type(4)));
   typedef uint32_t u2 __attribute__((ext_vector_type(2)));
   typedef typename std::conditional<W == 16, u4, u2>::type vec;
   constexpr uint64_t TILE = (uint64_t)LANES * W * LOADS;
   const uint32_t off = threadIdx.x * (uint32_t)W;
#pragma unroll 1
   for(uint32_t i = 0; i < per; i++) {
      const uint64_t tile = stride ? (uint64_t)blockIdx.x + (uint64_t)i * gridDim.x
                                   : (uint64_t)blockIdx.x * per + i;
      if(tile >= tiles) break;
      const uint64_t base = tile * TILE;
      const uint64_t left = bytes - base;
      const uint32_t size = left < TILE ? (uint32_t)left : (uint32_t)TILE;
      const __amdgpu_buffer_rsrc_t ri =
         __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(in) + base, 0, (int)size, Buf::kFlags);
      const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(out + base, 0, (int)size, Buf::kFlags);
      vec v[LOADS];
#pragma unroll
      for(int u = 0; u < LOADS; u++) {
         if constexpr(W == 16) v[u] = __builtin_amdgcn_raw_buffer_load_b128(ri, off, u * LANES * W, PLD);
         else                  v[u] = __builtin_amdgcn_raw_buffer_load_b64(ri, off, u * LANES * W, PLD);
      }
#pragma unroll
      for(int u = 0; u < LOADS; u++) {
         if constexpr(W == 16) __builtin_amdgcn_raw_buffer_store_b128(v[u], ro, off, u * LANES * W, PST);
         else                  __builtin_amdgcn_raw_buffer_store_b64(v[u], ro, off, u * LANES * W, PST);
      }
   }
}

template<int LANES, int W, int LOADS, int PLD>
const void* pick_store(int pst)
{
   switch(pst) {
      case 0:  return reinterpret_cast<const void*>(&stream_kernel<LANES, W, LOADS, PLD, 0>);
      case 1:  return reinterpret_cast<const void*>(&stream_kernel<LANES, W, LOADS, PLD, 1>);
      case 2:  return reinterpret_cast<const void*>(&stream_kernel<LANES, W, LOADS, PLD, 2>);
      default: return reinterpret_cast<const void*>(&stream_kernel<LANES, W, LOADS, PLD, 3>);
   }
}

template<int LANES, int W, int LOADS>
const void* pick_load(int pld, int pst)
{
   // 1024 lanes are 4 waves per SIMD: 128 VGPRs a lane, which 512 bytes of
   // loads in flight would fill (the compiler spills)
   if constexpr(LANES * W * LOADS > 256 * 1024) {
      return nullptr;
   } else {
      switch(pld) {
         case 0:  return pick_store<LANES, W, LOADS, 0>(pst);
         case 1:  return pick_store<LANES, W, LOADS, 1>(pst);
         case 2:  return pick_store<LANES, W, LOADS, 2>(pst);
         default: return pick_store<LANES, W, LOADS, 3>(pst);
      }
   }
}

template<int LANES, int W>
const void* pick_loads(int loads, int pld, int pst)
{
   switch(loads) {
      case 1:  return pick_load<LANES, W, 1>(pld, pst);
      case 2:  return pick_load<LANES, W, 2>(pld, pst);
      case 4:  return pick_load<LANES, W, 4>(pld, pst);
      case 8:  return pick_load<LANES, W, 8>(pld, pst);
      case 16: return pick_load<LANES, W, 16>(pld, pst);
      default: return pick_load<LANES, W, 32>(pld, pst);
   }
}

template<int LANES>
const void* pick(int width, int loads, int pld, int pst)
{
   return width == 16 ? pick_loads<LANES, 16>(loads, pld, pst) : pick_loads<LANES, 8>(loads, pld, pst);
}

}  // namespace

bool stream_shape_ok(int lanes, int width, int loads, int per, int groups, int pld, int pst)
{
   return (lanes == 64 || lanes == 256 || lanes == 1024) && (width == 8 || width == 16) && loads >= 1 &&
          loads <= 32 && (loads & (loads - 1)) == 0 && lanes * width * loads <= 256 * 1024 && per >= 1 &&
          per <= 4096 && groups >= 0 && pld >= 0 && pld <= 3 && pst >= 0 && pst <= 3;
}

hipError_t launch_stream_shape(const void* in, void* out, uint64_t bytes, int lanes, int width, int loads,
                               int per, int groups, int pld, int pst, hipStream_t s)
{
   if(!stream_shape_ok(lanes, width, loads, per, groups, pld, pst)) return hipErrorInvalidValue;
   if(bytes == 0) return hipSuccess;
   const uint64_t tb = (uint64_t)lanes * (uint64_t)width * (uint64_t)loads;
   const uint64_t tiles = (bytes + tb - 1) / tb;
   uint64_t grid = 0;
   uint32_t p = (uint32_t)per, stride = 0;
   if(groups > 0) {
      // persistent: `groups` workgroups (at most one per tile) stride over the tiles
      grid = (uint64_t)groups < tiles ? (uint64_t)groups : tiles;
      p = (uint32_t)((tiles + grid - 1) / grid);
      stride = 1;
   } else {
      grid = (tiles + p - 1) / p;
   }
   if(grid > 0x7fffffffull) return hipErrorInvalidValue;
   const void* k = lanes == 64 ? pick<64>(width, loads, pld, pst)
                 : lanes == 256 ? pick<256>(width, loads, pld, pst) : pick<1024>(width, loads, pld, pst);
   if(!k) return hipErrorInvalidValue;
   const char* pi = static_cast<const char*>(in);
   char* po = static_cast<char*>(out);
   uint64_t b = bytes, t = tiles;
   void* argv[] = { &pi, &po, &b, &t, &p, &stride };
   return hipLaunchKernel(k, dim3((unsigned)grid), dim3((unsigned)lanes), argv, 0, s);
}

// the fixed shape of fufft_stream_f32: 256 lanes, eight 16-byte loads per
// lane, one 32 KiB tile per workgroup, NT on both sides or on neither
hipError_t launch_stream(const void* in, void* out, uint64_t bytes, bool nontemporal, hipStream_t s)
{
   const int pol = nontemporal ? kNT : 0;
   return launch_stream_shape(in, out, bytes, 256, 16, 8, 1, 0, pol, pol, s);
}

}  // namespace fufft
