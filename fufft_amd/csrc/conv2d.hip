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
         const uint32_t fo = (uint32_t)(L * V) * W8 + fc * 8u;
         // The split apply with one filter per image reads each filter once:
         // in the library's column order its tiles stream past the caches
         // (NT), which leaves them to the shared spectrum; 512 x 512 x 256
         // filters +3.9% (same box).  In the reference's order a tile's
         // columns are scattered over the row, its cache lines are shared
         // with other tiles, and NT cost 4.5%.
         if constexpr(KIND == COL_APPLY) {
            if(!p.f_dr && p.fcount == p.nimg) mid_op<PL, MID, POL_NT>(r, fb, fo, W8);
            else                              mid_op<PL, MID>(r, fb, fo, W8);
         } else {
            mid_op<PL, MID>(r, fb, fo, W8);
         }
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

// ---- small images: the whole 2D conv in one workgroup ------------------------------------
// fufft_conv2d<H, W, CPB> (fufft.cuh:1209-1258; its transcription kernel_conv2d,
// verify_kernel.cpp:700-722) for images of H x W <= 8192 points, H and W powers
// of two from 8 to 512: rows DIF, columns DIF, mid, columns DIT, rows DIT, every
// step through LDS, radix 8 both ways (the reference's per-dimension plans), so
// with the reference's base twiddles the result is its transcription's bit for
// bit.  An image has I = H*W/8 lanes.  In the row phases lane i runs row i / TW
// at lane i % TW (TW = W/8), in the column phases column i / TH at lane i % TH
// (TH = H/8); both are at most 64, so each row or column transform lies inside
// one wavefront and its exchanges need a wavefront fence only.  Between the
// phases the image crosses LDS transposed (columns contiguous, one spare slot
// per column); workgroup barriers order those crossings.  Images past the
// batch run on empty buffer ranges (loads return zero, stores are dropped), so
// every lane meets every barrier.
constexpr int small2d_lanes(int h, int w) { return h * w / 8; }
constexpr int small2d_images(int h, int w) { return small2d_lanes(h, w) >= 256 ? 1 : 256 / small2d_lanes(h, w); }
constexpr int small2d_slot(int h, int w)
{
   const int rows = h * (w + w / 8), cols = w * (h + h / 8), tr = w * (h + 1);
   return rows > cols ? (rows > tr ? rows : tr) : (cols > tr ? cols : tr);
}

template<int H, int W, int MID>
__global__ void __launch_bounds__(small2d_images(H, W) * small2d_lanes(H, W))
small2d_kernel(const Small2dParams p)
{
   using PW = Plan<W, 8>;
   using PH = Plan<H, 8>;
   using LD = Lds<8, LAYOUT_PAD>;
   using Op = MidOf<MID>;
   constexpr int TW = W / 8, TH = H / 8, I = small2d_lanes(H, W), IPB = small2d_images(H, W);
   constexpr int SW = LD::size(W), SH = LD::size(H), CT = H + 1, SLOT = small2d_slot(H, W);
   constexpr uint32_t BYTES = H * W * 8;
   static_assert(TW <= 64 && TH <= 64, "a row or column transform inside one wavefront");

   extern __shared__ float2 lds[];
   const int img = threadIdx.x / I, i = threadIdx.x % I;
   const uint32_t t = blockIdx.x * IPB + img;
   const bool live = t < p.nimg;
   float2* S = lds + img * SLOT;
   const int rr = i / TW, rl = i % TW;            // row phases: row, lane in the row
   const int cc = i / TH, cl = i % TH;            // column phases: column, lane in the column

   Twiddles<PW> tww;
   tww.load(p.tw, rl);
   Twiddles<PH> twh;
   twh.load(p.tw, cl);

   // Rows of at most 16 points (128 bytes), or 32 in images of at most 2048
   // points: a wavefront's row-wise 8-byte loads would touch 16-32 cache
   // lines per instruction.  Instead every
   // wavefront loads its own 512 points (its lanes' 8 each, consecutive in
   // the batch) with one contiguous 512-byte run per instruction and passes
   // them through its rows' LDS (row stride SW) to the lanes that transform
   // them; the result leaves the same way.  A row's lanes, and the LDS row
   // they use, belong to one wavefront, so a wavefront fence orders the
   // hand-over.  Points past the batch read as zero and are not written.
   // Same box, Gpt/s before -> after: 8 x 8 116 -> 371, 32 x 8 145 -> 314,
   // 512 x 8 153 -> 228, 16 x 16 182 -> 328, 512 x 16 139 -> 156, 32 x 32
   // 240 -> 288, 64 x 32 253 -> 281; at 128 x 32 and 256 x 32 the extra
   // registers cost a workgroup per CU (238 -> 235, 227 -> 216) and at 64
   // points per row the row loads already use half of each line (64 x 64
   // 269 -> 259), so those keep the direct loads.
   constexpr bool STAGE = W <= 16 || (W == 32 && H * W <= 2048);
   const uint32_t wv = threadIdx.x / 64, wl = threadIdx.x % 64;
   const uint64_t wp = ((uint64_t)blockIdx.x * IPB * I + wv * 64u) * 8u;   // wavefront's first point
   const uint64_t total = (uint64_t)p.nimg * (H * W);
   const uint32_t wbytes = wp >= total ? 0u : (uint32_t)((total - wp < 512u ? total - wp : 512u) * 8u);
   // LDS slot of the wavefront's point lp: image, row and column of its index in the workgroup
   auto stage_slot = [&](uint32_t lp) {
      const uint32_t g = wv * 512u + lp, im = g / (H * W), pt = g % (H * W);
      return im * SLOT + (pt / W) * SW + pt % W;
   };

   // rows DIF: lane (rr, rl) takes row rr's points rl + q*TW; leaves its row's
   // spectrum slots rl*8 + k in registers
   float2 r[8];
   if constexpr(STAGE) {
      const Buf wb(static_cast<const char*>(p.in) + wp * 8u, wbytes);
      float2 v[8];
#pragma unroll
      for(int q = 0; q < 8; q++) v[q] = wb.ld2(wl * 8u, q * 512);
#pragma unroll
      for(int q = 0; q < 8; q++) lds[stage_slot(q * 64 + wl)] = v[q];
      pass_barrier<64>();
#pragma unroll
      for(int q = 0; q < 8; q++) r[q] = S[rr * SW + rl + q * TW];
   } else {
      const Buf ib(static_cast<const char*>(p.in) + (size_t)t * BYTES, live ? BYTES : 0u);
#pragma unroll
      for(int q = 0; q < 8; q++) r[q] = ib.ld2((uint32_t)(rr * W + rl) * 8u, q * TW * 8);
   }
   forward_dif<PW, LD, 64>(r, S + rr * SW, rl, tww);
   // transposed: row-spectrum slot s of row rr to S[s*CT + rr]
   __syncthreads();
#pragma unroll
   for(int k = 0; k < 8; k++) S[(rl * 8 + k) * CT + rr] = r[k];
   __syncthreads();
   // columns DIF: lane (cc, cl) takes column cc's rows cl + q*TH
#pragma unroll
   for(int q = 0; q < 8; q++) r[q] = S[cc * CT + cl + q * TH];
   __syncthreads();
   KeptChain<PH> kc;
   forward_dif<PH, LD, 64, 64, KEEP_STORE>(r, S + cc * SH, cl, twh, kc);
   // mid: column-spectrum slot cl*8 + k of column cc is 2D slot (cl*8 + k, cc)
   if constexpr(Op::reads_filter) {
      const uint32_t fi = modulo_count(t, p.fcount);
      const Buf fb(static_cast<const char*>(p.filt) + (size_t)fi * BYTES, live ? BYTES : 0u);
      float2 b[8];
      if constexpr(H >= 64 && H * W <= 4096) {
         // A lane's filter values run down its column, W points apart, and a
         // wavefront's TH = H/8 lanes per column read TH rows at once, so from
         // 64 rows on one wavefront instruction touches 8-64 cache lines.  In
         // these images each wavefront lies in one image and loads 512
         // consecutive filter points instead (512-byte runs),
         // after a barrier writes them into their columns' LDS (entry (r, c)
         // at c*SH + (r + r/8 + c) mod SH: 9 slots per lane's 8 rows and a
         // turn per column, so both sides stay nearly free of bank conflicts),
         // and after a second barrier each lane reads its 8 rows.  A column's
         // LDS is read and then reused by its own lanes only, so the inverse
         // needs no third barrier.  Same box, Gpt/s before -> after: 512 x 8
         // 229 -> 274, 64 x 64 281 -> 293, 128 x 32 248 -> 263, 256 x 16 241 ->
         // 251, 64 x 8 321 -> 335, 64 x 32 291 -> 283; at 8192 points the two
         // arrays it holds across the barrier cost a workgroup per CU (128 x 64
         // 224 -> 174, 256 x 32 235 -> 192), and with fewer than 64 rows the
         // direct reads take 1-4 cache lines per instruction (32 x 32 298 ->
         // 278, 8 x 512 277 -> 258), so those read in place.
         const uint32_t pt0 = (wv * 512u) % (H * W);
         float2 v[8];
#pragma unroll
         for(int q = 0; q < 8; q++) v[q] = fb.ld2((pt0 + wl) * 8u, q * 512);
         __syncthreads();                          // every column's forward DIF is done with S
#pragma unroll
         for(int q = 0; q < 8; q++) {
            const uint32_t pt = pt0 + q * 64 + wl, row = pt / W, col = pt % W;
            S[col * SH + (row + row / 8 + col) % SH] = v[q];
         }
         __syncthreads();
#pragma unroll
         for(int k = 0; k < 8; k++) b[k] = S[cc * SH + (cl * 9 + k + cc) % SH];
      } else {
#pragma unroll
         for(int k = 0; k < 8; k++) b[k] = fb.ld2((uint32_t)(cl * 8 * W + cc) * 8u, k * W * 8);
      }
#pragma unroll
      for(int k = 0; k < 8; k++) r[k] = Op::apply(r[k], b[k]);
   } else {
#pragma unroll
      for(int k = 0; k < 8; k++) r[k] = Op::apply(r[k], make_float2(0.f, 0.f));
   }
   inverse_dit<PH, LD, 64, 64, KEEP_USE>(r, S + cc * SH, cl, twh, kc);
   // transposed back: column cc's rows cl + q*TH to S[cc*CT + row]
   __syncthreads();
#pragma unroll
   for(int q = 0; q < 8; q++) S[cc * CT + cl + q * TH] = r[q];
   __syncthreads();
   // rows DIT: lane (rr, rl) takes row rr's spectrum slots rl*8 + k
#pragma unroll
   for(int k = 0; k < 8; k++) r[k] = S[(rl * 8 + k) * CT + rr];
   __syncthreads();
   inverse_dit<PW, LD, 64>(r, S + rr * SW, rl, tww);
   if constexpr(STAGE) {
#pragma unroll
      for(int q = 0; q < 8; q++) S[rr * SW + rl + q * TW] = r[q];
      pass_barrier<64>();
      const Buf wb(static_cast<char*>(p.out) + wp * 8u, wbytes);
#pragma unroll
      for(int q = 0; q < 8; q++) wb.st2(lds[stage_slot(q * 64 + wl)], wl * 8u, q * 512);
   } else {
      const Buf ob(static_cast<char*>(p.out) + (size_t)t * BYTES, live ? BYTES : 0u);
#pragma unroll
      for(int q = 0; q < 8; q++) ob.st2(r[q], (uint32_t)(rr * W + rl) * 8u, q * TW * 8);
   }
}

template<int H, int W, int MID>
static hipError_t launch_small2d_one(const Small2dParams& p, hipStream_t s)
{
   constexpr int IPB = small2d_images(H, W);
   const size_t shm = (size_t)IPB * small2d_slot(H, W) * sizeof(float2);
   const void* k = reinterpret_cast<const void*>(&small2d_kernel<H, W, MID>);
   if(!modulo_count_ok(p.fcount, p.nimg)) return hipErrorInvalidValue;
   static std::atomic<uint64_t> lds_ok{0};
   if(const hipError_t e = ensure_dynamic_lds(k, shm, lds_ok); e != hipSuccess) return e;
   const dim3 grid((p.nimg + IPB - 1) / IPB), block(IPB * small2d_lanes(H, W));
   Small2dParams arg = p;
   void* argv[] = { &arg };
   return hipLaunchKernel(k, grid, block, argv, shm, s);
}

template<int H, int W>
static hipError_t launch_small2d_hw(const Small2dParams& p, hipStream_t s)
{
   if constexpr(H * W <= 8192)
      return with_mid(p.mid, [&](auto m) { return launch_small2d_one<H, W, decltype(m)::value>(p, s); });
   else
      return hipErrorInvalidValue;
}

template<int H>
static hipError_t launch_small2d_h(int w, const Small2dParams& p, hipStream_t s)
{
   switch(w) {
      case 8:   return launch_small2d_hw<H, 8>(p, s);
      case 16:  return launch_small2d_hw<H, 16>(p, s);
      case 32:  return launch_small2d_hw<H, 32>(p, s);
      case 64:  return launch_small2d_hw<H, 64>(p, s);
      case 128: return launch_small2d_hw<H, 128>(p, s);
      case 256: return launch_small2d_hw<H, 256>(p, s);
      case 512: return launch_small2d_hw<H, 512>(p, s);
      default:  return hipErrorInvalidValue;
   }
}

bool small2d_supported(int64_t h, int64_t w)
{
   const bool ph = h >= 8 && h <= 512 && (h & (h - 1)) == 0, pw = w >= 8 && w <= 512 && (w & (w - 1)) == 0;
   return ph && pw && h * w <= 8192;
}

hipError_t launch_small2d(int h, int w, const Small2dParams& p, hipStream_t s)
{
   switch(h) {
      case 8:   return launch_small2d_h<8>(w, p, s);
      case 16:  return launch_small2d_h<16>(w, p, s);
      case 32:  return launch_small2d_h<32>(w, p, s);
      case 64:  return launch_small2d_h<64>(w, p, s);
      case 128: return launch_small2d_h<128>(w, p, s);
      case 256: return launch_small2d_h<256>(w, p, s);
      case 512: return launch_small2d_h<512>(w, p, s);
      default:  return hipErrorInvalidValue;
   }
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
