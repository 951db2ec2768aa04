// 2D column kernels for gfx950.
//
// A 2D conv runs, in the reference's order (verify_kernel.cpp:700-722), rows
// DIF -> columns DIF -> mid -> columns DIT -> rows DIT.  An image of 512 x 512
// complex points is 2 MiB, more than a workgroup's LDS, so the rows are done by
// the 1D kernels (forward into digit order, inverse from digit order) and the
// columns by the kernels here: each workgroup takes C adjacent columns of one
// image through the column DIF, the mid operation and the column DIT.
// Replaces fufft_col_pass / fufft_conv2d (fufft.cuh:1185-1258), which only fit
// H*W <= 4096 in one block.
//
// Mapping: thread = (lane L of the column transform, column col) with the
// column fastest, so every tap load or store of a wavefront covers 64/C rows
// of C consecutive points -- full 128-byte runs for C = 16.  Each column keeps
// its own LDS slot.  The exchanges are ds_read2_b64 / ds_write2_b64, and
// gfx950 services each of their 8-byte accesses 16 lanes at a time: lanes of
// one quarter-wavefront conflict when their float2 slots agree modulo 16
// (measured with SQ_LDS_BANK_CONFLICT; tests/test_lds_audit.py).  A quarter
// holds 16/C lanes L of C columns, so slots are skewed by 16/C float2 (the
// padded slot size is a multiple of 16): the columns then fall on distinct
// residues, and every exchange is conflict-free.
#include "fufft_device.hpp"
#include "fufft_plan.hpp"
#include "fufft_internal.hpp"

namespace fufft {

// values per lane and columns per workgroup for a column length h
constexpr int col_v(int h) { return h <= 512 ? 8 : 16; }
constexpr int col_c(int h) { return (1024 / (h / col_v(h))) < 16 ? 1024 / (h / col_v(h)) : 16; }

template<int H, int V, int LAYOUT, int KIND, int MID, int C>
__global__ void __launch_bounds__(C * (H / V)) col_kernel(const ColParams p)
{
   using PL = Plan<H, V>;
   using LD = Lds<V, LAYOUT>;
   constexpr int T     = PL::T;
   constexpr int SLOTC = LD::size(H) + 16 / C;

   extern __shared__ float2 lds[];
   const int col = threadIdx.x % C;
   const int L   = threadIdx.x / C;
   const uint32_t tiles = p.w / C;
   const uint32_t img   = blockIdx.x / tiles;
   const uint32_t c     = (blockIdx.x - img * tiles) * C + col;
   const uint32_t W8    = p.w * 8u;
   const uint32_t ibytes = (uint32_t)H * W8;
   const uint32_t nat = (uint32_t)L * W8 + c * 8u;           // row L, column c
   const uint32_t dro = (uint32_t)(L * V) * W8 + c * 8u;     // row slot L*V, column c

   float2* A = lds + col * SLOTC;
   Twiddles<PL> tw;
   tw.load(p.tw, L);
   constexpr int KEEP_F = KIND == COL_CONV ? KEEP_STORE : KEEP_NONE;
   constexpr int KEEP_I = KIND == COL_CONV ? KEEP_USE : KEEP_NONE;
   KeptChain<PL> kc;
   float2 r[V];

   if constexpr(KIND == COL_APPLY) {
      const Buf sb(static_cast<const char*>(p.spec) + (size_t)modulo_count(img, p.scount) * ibytes, ibytes);
#pragma unroll
      for(int k = 0; k < V; k++) r[k] = sb.ld2(dro, k * W8);
   } else {
      const Buf ib(static_cast<const char*>(p.in) + (size_t)img * ibytes, ibytes);
#pragma unroll
      for(int q = 0; q < V; q++) r[q] = ib.ld2(nat, q * T * W8);
      forward_dif<PL, LD, C * T, 64 / C, KEEP_F>(r, A, L, tw, kc);
   }

   const Buf ob(static_cast<char*>(p.out) + (size_t)img * ibytes, ibytes);
   if constexpr(KIND == COL_FWD) {
#pragma unroll
      for(int k = 0; k < V; k++) ob.st2(r[k], dro, k * W8);
   } else {
      {
         const Buf fb(static_cast<const char*>(p.filt) + (size_t)modulo_count(img, p.fcount) * ibytes, ibytes);
         const uint32_t fc = p.f_dr ? lane_slot(c, p.f_tr_log, p.f_vr_log) : c;
         mid_op<PL, MID>(r, fb, (uint32_t)(L * V) * W8 + fc * 8u, W8);
      }
      inverse_dit<PL, LD, C * T, 64 / C, KEEP_I>(r, A, L, tw, kc);
#pragma unroll
      for(int q = 0; q < V; q++) ob.st2(r[q], nat, q * T * W8);
   }
}

template<int H, int KIND, int MID>
static hipError_t launch_col_one(const ColParams& p, hipStream_t s)
{
   constexpr int V = col_v(H), T = H / V, C = col_c(H);
   constexpr int SLOTC = Lds<V, LAYOUT_PAD>::size(H) + 16 / C;
   const size_t shm = (size_t)C * SLOTC * sizeof(float2);
   const void* k = reinterpret_cast<const void*>(&col_kernel<H, V, LAYOUT_PAD, KIND, MID, C>);
   static std::atomic<uint64_t> lds_ok{0};
   if(const hipError_t e = ensure_dynamic_lds(k, shm, lds_ok); e != hipSuccess) return e;
   if(p.w % C || !modulo_count_ok(p.fcount, p.nimg) || !modulo_count_ok(p.scount, p.nimg))
      return hipErrorInvalidValue;
   const uint64_t blocks = (uint64_t)p.nimg * (p.w / C);
   if(blocks > 0x7fffffffu) return hipErrorInvalidValue;
   const dim3 grid((unsigned)blocks), block(C * T);
   ColParams arg = p;
   void* argv[] = { &arg };
   return hipLaunchKernel(k, grid, block, argv, shm, s);
}

template<int H, int KIND>
static hipError_t launch_col_mid(const ColParams& p, hipStream_t s)
{
   if constexpr(KIND == COL_FWD) {
      return launch_col_one<H, KIND, MID_NONE>(p, s);
   } else {
      return with_mid(p.mid, [&](auto m) { return launch_col_one<H, KIND, decltype(m)::value>(p, s); });
   }
}

template<int H>
static hipError_t launch_col_h(int kind, const ColParams& p, hipStream_t s)
{
   switch(kind) {
      case COL_CONV:  return launch_col_mid<H, COL_CONV>(p, s);
      case COL_FWD:   return launch_col_mid<H, COL_FWD>(p, s);
      case COL_APPLY: return launch_col_mid<H, COL_APPLY>(p, s);
      default:        return hipErrorInvalidValue;
   }
}

int col_values_per_lane(int h)
{
   return (h == 256 || h == 512 || h == 1024 || h == 2048) ? col_v(h) : 0;
}

hipError_t launch_col(int kind, int h, const ColParams& p, hipStream_t s)
{
   switch(h) {
      case 256:  return launch_col_h<256>(kind, p, s);
      case 512:  return launch_col_h<512>(kind, p, s);
      case 1024: return launch_col_h<1024>(kind, p, s);
      case 2048: return launch_col_h<2048>(kind, p, s);
      default:   return hipErrorInvalidValue;
   }
}

}  // namespace fufft
