// C-ABI layer: argument checking, host planning, the device twiddle table and
// dispatch to the kernel translation units.  Declarations and the reference
// interfaces each entry point replaces are in include/fufft/fufft.h.
#include "fufft_internal.hpp"
#include "fufft_plan.hpp"
#include "../../include/fufft/fufft.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

namespace fufft {

// ---- twiddle table ----------------------------------------------------------------
// Static device memory: every GPU the library runs on holds one copy, filled
// once by fufft_init.  Level P = 2^p (1 <= p <= FUFFT_TW_LOG_MAX) occupies
// entries [P, 2P): (cos, sin)(2*pi*t/P) rounded to fp32 by default, or, with
// fufft_set_twiddles(FUFFT_TWIDDLES_REFERENCE), the reference's fp32-angle
// values.
__device__ float2 g_twiddle[FUFFT_TW_ENTRIES];

// Scratch of fufft_conv2d_r2_noalloc_f32: the packed complex images of one
// sub-batch, in place of a caller workspace.  Every GPU the library runs on
// holds one copy until the process ends.  In host code this name stands for
// no device address: init_device() looks up each device's copy with
// hipGetSymbolAddress and keeps it in DeviceState::scratch, and only that
// address reaches the kernels.
static __device__ __align__(256) float2 scratch[FUFFT_SCRATCH_BYTES / sizeof(float2)];

namespace {

constexpr int kMaxDevices = 64;

struct DeviceState {
   std::atomic<int> ready{0};
   std::atomic<int> source{FUFFT_TWIDDLES_ACCURATE};
   const float2*    tw = nullptr;
   float2*          scratch = nullptr;   // this device's copy of `scratch`
};
DeviceState g_dev[kMaxDevices];
std::mutex  g_init_mutex;

// (cos, sin)(2*pi*t/P) in double, rounded to float.  The CPU oracle
// (oracle/oracle.c: table_cs) evaluates this same expression.
void table_entry(int P, int64_t t, float* c, float* s)
{
   const double th = 6.283185307179586476925286766559 * (double)t / (double)P;
   *c = (float)cos(th);
   *s = (float)sin(th);
}

// The reference's base twiddle: cosf / sinf of the fp32 angle step * j with
// step = 2*pi/P in fp32 (verify_kernel.cpp:31, 93, 99; the device code's
// __sincosf(step * j), fufft.cuh:362-371).  The forward passes use
// step = -2*pi/P; that angle is the exact negation of this one and libm's
// cosf / sinf are even / odd bit for bit, so negating the stored sine gives
// the forward twiddle exactly as the reference computes it.
void table_entry_reference(int P, int64_t t, float* c, float* s)
{
   const float step = 6.28318530717958647692f / (float)P;
   const float ang  = step * (float)t;
   *c = cosf(ang);
   *s = sinf(ang);
}

void fill_table(int log_max, float* out, int source = FUFFT_TWIDDLES_ACCURATE)
{
   out[0] = out[1] = out[2] = out[3] = 0.0f;
   for(int p = 1; p <= log_max; p++) {
      const int P = 1 << p;
      for(int t = 0; t < P; t++) {
         float* e = &out[2 * (P + t)];
         if(source == FUFFT_TWIDDLES_REFERENCE) table_entry_reference(P, t, e, e + 1);
         else                                   table_entry(P, t, e, e + 1);
      }
   }
}

// Fill the whole table from `source` and copy it to the current device
// (synchronous).  Returns the table's device address through addr.
int upload_table(int source, void** addr)
{
   std::vector<float> host(2 * (size_t)FUFFT_TW_ENTRIES);
   fill_table(FUFFT_TW_LOG_MAX, host.data(), source);
   if(hipMemcpyToSymbol(HIP_SYMBOL(g_twiddle), host.data(), host.size() * sizeof(float), 0,
                        hipMemcpyHostToDevice) != hipSuccess ||
      hipGetSymbolAddress(addr, HIP_SYMBOL(g_twiddle)) != hipSuccess || *addr == nullptr)
      return FUFFT_ERR_HIP;
   return FUFFT_OK;
}

// LDS layout: each plan's additive default (per-exchange layouts, or the
// padded one; default_lds_layout) unless FUFFT_LDS_LAYOUT=xor selects the
// zero-padding XOR swizzle (a tuning knob; all are bit-identical)
int lds_layout()
{
   static const int layout = [] {
      const char* e = std::getenv("FUFFT_LDS_LAYOUT");
      return (e && std::strcmp(e, "xor") == 0) ? LAYOUT_XOR : LAYOUT_DEFAULT;
   }();
   return layout;
}

// Items (transforms, images) per sub-batch of the multi-launch paths (four-
// step, 2D), for item_bytes per item.  A sub-batch about the size of MI355X's
// last-level (Infinity) cache, 256 MiB, keeps the data one launch writes
// resident for the next launch.  Measured (Gpt/s or G px/s at 32 / 64 / 128 /
// 192 / 256 MiB): four-step N = 32768 98 / 113 / 124 / 128 / 131 (109 without
// sub-batches); 2D 512^2 two-for-one 170 / 197 / 214 / 210 / 201, whose
// launches touch two arrays of the sub-batch's size (two real inputs and a
// complex work array), so it runs at 128 MiB.  FUFFT_SUBBATCH_MB overrides
// both; 0 disables sub-batching.
enum { SUBBATCH_FOURSTEP_MB = 256, SUBBATCH_2D_MB = 128 };

int64_t subbatch_items(int64_t item_bytes, int64_t batch, int64_t default_mb)
{
   static const int64_t env_mb = [] {
      const char* e = std::getenv("FUFFT_SUBBATCH_MB");
      return e ? (int64_t)std::atoll(e) : (int64_t)-1;
   }();
   const int64_t mb = env_mb >= 0 ? env_mb : default_mb;
   if(mb <= 0) return batch > 0 ? batch : 1;
   const int64_t items = (mb << 20) / item_bytes;
   return items > 0 ? items : 1;
}

int init_device(int dev)
{
   if(dev < 0 || dev >= kMaxDevices) return FUFFT_ERR_INVALID;
   DeviceState& d = g_dev[dev];
   if(d.ready.load(std::memory_order_acquire)) return FUFFT_OK;
   std::lock_guard<std::mutex> lock(g_init_mutex);
   if(d.ready.load(std::memory_order_relaxed)) return FUFFT_OK;

   int prev = 0;
   if(hipGetDevice(&prev) != hipSuccess) return FUFFT_ERR_HIP;
   if(prev != dev && hipSetDevice(dev) != hipSuccess) return FUFFT_ERR_HIP;
   void* addr = nullptr;
   int status = upload_table(FUFFT_TWIDDLES_ACCURATE, &addr);
   float2* sp = nullptr;
   if(status == FUFFT_OK &&
      (hipGetSymbolAddress((void**)&sp, HIP_SYMBOL(scratch)) != hipSuccess || sp == nullptr))
      status = FUFFT_ERR_HIP;
   if(prev != dev) (void)hipSetDevice(prev);
   if(status != FUFFT_OK) return status;
   d.tw = static_cast<const float2*>(addr);
   d.scratch = sp;
   d.source.store(FUFFT_TWIDDLES_ACCURATE, std::memory_order_relaxed);
   d.ready.store(1, std::memory_order_release);
   return FUFFT_OK;
}

int set_twiddles(int dev, int source)
{
   if(source != FUFFT_TWIDDLES_ACCURATE && source != FUFFT_TWIDDLES_REFERENCE) return FUFFT_ERR_INVALID;
   const int st = init_device(dev);
   if(st != FUFFT_OK) return st;
   DeviceState& d = g_dev[dev];
   std::lock_guard<std::mutex> lock(g_init_mutex);
   if(d.source.load(std::memory_order_relaxed) == source) return FUFFT_OK;
   int prev = 0;
   if(hipGetDevice(&prev) != hipSuccess) return FUFFT_ERR_HIP;
   if(prev != dev && hipSetDevice(dev) != hipSuccess) return FUFFT_ERR_HIP;
   // kernels already queued on any stream read the table: let them finish first
   int status = hipDeviceSynchronize() == hipSuccess ? FUFFT_OK : FUFFT_ERR_HIP;
   void* addr = nullptr;
   if(status == FUFFT_OK) status = upload_table(source, &addr);
   if(prev != dev) (void)hipSetDevice(prev);
   if(status == FUFFT_OK) d.source.store(source, std::memory_order_relaxed);
   return status;
}

// twiddle table (and scratch) of the current device, initialising it on first use
int current_table(const float2** tw, float2** scr = nullptr)
{
   int dev = 0;
   if(hipGetDevice(&dev) != hipSuccess) return FUFFT_ERR_HIP;
   const int st = init_device(dev);
   if(st != FUFFT_OK) return st;
   *tw = g_dev[dev].tw;
   if(scr) *scr = g_dev[dev].scratch;
   return FUFFT_OK;
}

int status_of(hipError_t e) { return e == hipSuccess ? FUFFT_OK : FUFFT_ERR_HIP; }

bool pow2(int64_t n) { return n > 0 && (n & (n - 1)) == 0; }

// the single-launch kernels' sizes (conv1d.hip): every 1D call
static bool single_supported(int64_t n, int v) { return pow2(n) && n <= 16384 && conv1d_supported((int)n, v); }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

// The device buffers of one call either coincide, where the call works in
// place, or share no byte.  A partial overlap would let one workgroup's (or
// one sub-batch's) stores land in data that another still has to read, so
// the entry points return FUFFT_ERR_INVALID for it.
struct Span {
   const void* p;
   uint64_t    bytes;
};

static bool disjoint(Span a, Span b)
{
   if(!a.p || !b.p || a.bytes == 0 || b.bytes == 0) return true;
   const uintptr_t x = reinterpret_cast<uintptr_t>(a.p), y = reinterpret_cast<uintptr_t>(b.p);
   return x + a.bytes <= y || y + b.bytes <= x;
}

// in place (the same bytes) or apart
static bool same_or_disjoint(Span a, Span b) { return (a.p == b.p && a.bytes == b.bytes) || disjoint(a, b); }

// bytes of a filter or spectrum argument: one (stride 0) or one per item
static uint64_t per_item_bytes(int64_t stride, int64_t batch, int64_t item_bytes)
{
   return (uint64_t)(stride == 0 ? 1 : batch) * (uint64_t)item_bytes;
}

// the real two-for-one conv's buffers (1D or 2D, items of `pts` points):
// u and v each in place of x or y or apart from both, u and v apart, the
// filter and a caller workspace apart from every other argument
static bool r2_buffers_ok(const float* x, const float* y, const void* filt, int64_t filt_stride, const float* u,
                          const float* v, const void* work, uint64_t work_bytes, int64_t pts, int64_t batch)
{
   const uint64_t b = (uint64_t)(pts * batch * 4);
   const Span sx{x, b}, sy{y, b}, su{u, b}, sv{v, b}, sf{filt, per_item_bytes(filt_stride, batch, pts * 8)};
   const Span sw{work, work_bytes};
   return same_or_disjoint(sx, su) && same_or_disjoint(sx, sv) && same_or_disjoint(sy, su) &&
          same_or_disjoint(sy, sv) && disjoint(su, sv) && disjoint(su, sf) && disjoint(sv, sf) &&
          disjoint(sw, sx) && disjoint(sw, sy) && disjoint(sw, su) && disjoint(sw, sv) && disjoint(sw, sf);
}

// The faster variant for an N and a filter layout, one rule for the fp32 and
// the BFP conv (a filter planned for one serves both).  Same box, 2^27
// points, Gpt/s radix 8 / radix 16:
//   digit order: fp32 N = 512 371 / 345, 1024 330 / 337, 2048 323 / 328,
//     4096 319 / 310, 8192 251-257 / 251-255; BFP N = 1024 406 / 424,
//     2048 384 / 386, 4096 365 / 368, 8192 303 / 287;
//   lane-major pairs: fp32 N = 512 373 / 361, 1024 336 / 355, 2048 334 / 354,
//     4096 323 / 331, 8192 256 / 279; BFP N = 4096 355 / 365.
// Radix 16 reads its 16 filter values per lane as 8 loads of 16 bytes; in
// digit order each of them touches 64 cache lines per wavefront, lane-major
// 8, and radix 16 (4 wavefronts per SIMD) hides that latency worse than
// radix 8 (8 per SIMD).
int fastest_variant(int64_t n, int layout)
{
   // the reference's bperm (lane-major, 8-byte loads) favours radix 16 from
   // N = 1024 as the pairs do (N = 4096: 324 / 312 Gpt/s radix 16 / radix 8)
   if(layout == FUFFT_LAYOUT_LANE || layout == FUFFT_LAYOUT_BPERM) return n == 512 ? FUFFT_R8 : FUFFT_V16;
   // digit order: one rule for every call a digit-order filter or spectrum
   // ties together.  At N = 4096 the fp32 conv alone runs radix 16 faster
   // (335 / 327 Gpt/s, its filter read staged through LDS), the BFP conv is
   // even (374 / 371) and the split apply runs radix 8 9% faster (367 / 338,
   // both with the spectrum read staged through LDS at radix 16), so radix 8
   // stays.  At N = 8192 radix 16 wins the fp32 conv (275 / 258), the split
   // apply (342 / 334) and the C2C (358 / 345), radix 8 the BFP conv (310 /
   // 297); the rule keeps radix 8 there, as filters planned at FUFFT_AUTO by
   // earlier builds expect
   return (n == 512 || n == 4096 || n == 8192) ? FUFFT_R8 : FUFFT_V16;
}

// FUFFT_AUTO: the faster variant for the digit-order filter (the default
// layout), also where a call has no layout argument
// filter layouts of the 1D calls: digit order, lane-major pairs, the reference's bperm
bool layout1d_ok(int layout)
{
   return layout == FUFFT_LAYOUT_DR || layout == FUFFT_LAYOUT_LANE || layout == FUFFT_LAYOUT_BPERM;
}

int resolve_variant(int64_t n, int variant)
{
   if(variant != FUFFT_AUTO) return variant;
   return fastest_variant(n, FUFFT_LAYOUT_DR);
}

// Values per lane of the four-step middle (N = 512 .. 4096 per chunk):
// FUFFT_V16 is the reference's own middle (run_large launches
// fufft_pipeline_v16 on the chunks, bench_fufft.cu:368-386), and FUFFT_AUTO
// takes it; FUFFT_R8 is the radix-8 middle (conv_foursteps_cfg with the
// radix-8 middle, verify_kernel.cpp:373-394).
int large_middle_v(int variant)
{
   return variant == FUFFT_R8 ? 8 : (variant == FUFFT_V16 || variant == FUFFT_AUTO) ? 16 : 0;
}

int values_per_lane(int variant)
{
   return variant == FUFFT_V16 ? 16 : variant == FUFFT_R8 ? 8 : 0;
}

// log2 of a power of two
int ilog2(int64_t x)
{
   int b = 0;
   while(((int64_t)1 << b) < x) b++;
   return b;
}

// Pass plan of an n-point transform at v values per lane: log2(n) bits are
// covered by radix-v passes of log2(v) bits each; the bits left over form one
// leading radix-2/4/8 pass, which runs first.  Returns the pass count.
// (the reference factorises the same way: cpu_mixed.cpp:36-49)
int factor(int64_t n, int v, int* radices)
{
   const int bits = ilog2(n), vbits = ilog2(v);
   int count = 0;
   if(bits % vbits) radices[count++] = 1 << (bits % vbits);
   for(int k = bits / vbits; k > 0; k--) radices[count++] = v;
   return count;
}

// Slot -> bin map of the DIF output: the index's digits, of the plan's radix
// widths, come out in reverse pass order.  Consuming idx from its least
// significant end (the last pass's digit) and shifting the result left as it
// grows puts that digit on top and the first pass's digit at the bottom.
// (the filter format of mixedrev_host, bench_fufft.cu:63-82)
int32_t group_reverse(int32_t idx, const int* radices, int np)
{
   int32_t bin = 0;
   for(int i = np - 1; i >= 0; i--) {
      const int b = ilog2(radices[i]);
      bin = (bin << b) | (idx & ((1 << b) - 1));
      idx >>= b;
   }
   return bin;
}

// in-place iterative radix-2 DFT in double (natural order), sign -1 = forward
void dft_f64(std::vector<double>& x, int64_t n, int sign)
{
   for(int64_t i = 1, j = 0; i < n; i++) {
      int64_t bit = n >> 1;
      for(; j & bit; bit >>= 1) j ^= bit;
      j ^= bit;
      if(i < j) { std::swap(x[2 * i], x[2 * j]); std::swap(x[2 * i + 1], x[2 * j + 1]); }
   }
   for(int64_t len = 2; len <= n; len <<= 1) {
      const int64_t half = len / 2;
      for(int64_t k = 0; k < half; k++) {
         const double th = 6.283185307179586476925286766559 * (double)k / (double)len;
         const double wr = cos(th), wi = sign * sin(th);
         for(int64_t i = 0; i < n; i += len) {
            const int64_t a = i + k, b = i + k + half;
            const double br = x[2 * b] * wr - x[2 * b + 1] * wi;
            const double bi = x[2 * b] * wi + x[2 * b + 1] * wr;
            x[2 * b]     = x[2 * a] - br;  x[2 * b + 1] = x[2 * a + 1] - bi;
            x[2 * a]     = x[2 * a] + br;  x[2 * a + 1] = x[2 * a + 1] + bi;
         }
      }
   }
}

// natural-order spectrum in double from taps or a given spectrum, 1/n folded
std::vector<double> spectrum_of(int64_t n, int filter_kind, int fold_inv_n, const float* in)
{
   std::vector<double> s(2 * (size_t)n);
   for(int64_t i = 0; i < 2 * n; i++) s[i] = in[i];
   if(filter_kind == FUFFT_FILTER_TAPS) dft_f64(s, n, -1);
   if(fold_inv_n)
      for(auto& v : s) v /= (double)n;
   return s;
}

}  // namespace
}  // namespace fufft

using namespace fufft;

extern "C" {

int fufft_abi_version(void) { return FUFFT_ABI_VERSION; }

int fufft_init(int device) { return init_device(device); }

int fufft_set_twiddles(int device, int source) { return set_twiddles(device, source); }

int fufft_get_twiddles(int device, int* source)
{
   if(!source) return FUFFT_ERR_INVALID;
   const int st = init_device(device);
   if(st != FUFFT_OK) return st;
   *source = g_dev[device].source.load(std::memory_order_relaxed);
   return FUFFT_OK;
}

const char* fufft_status_string(int status)
{
   switch(status) {
      case FUFFT_OK:              return "ok";
      case FUFFT_ERR_INVALID:     return "invalid argument";
      case FUFFT_ERR_UNSUPPORTED: return "unsupported size or variant";
      case FUFFT_ERR_HIP:         return "HIP runtime error";
      case FUFFT_ERR_ALIGN:       return "misaligned pointer (16 bytes for fp32 data, 4 for BFP data)";
      case FUFFT_ERR_SCRATCH:     return "one image needs more than the static scratch (FUFFT_SCRATCH_BYTES)";
      default:                    return "unknown status";
   }
}

int fufft_supported(int64_t n, int variant)
{
   const int v = values_per_lane(resolve_variant(n, variant));
   return (v && (single_supported(n, v) || conv_wide_plan(n, v))) ? 1 : 0;
}

int fufft_fastest_variant(int64_t n, int layout)
{
   if(!layout1d_ok(layout)) return FUFFT_ERR_INVALID;
   if(!pow2(n) || n < 256 || n > CONV_WIDE_N) return FUFFT_ERR_UNSUPPORTED;
   return fastest_variant(n, layout);
}

int fufft_mid_reads_filter(int mid)
{
   if(!mid_known(mid)) return FUFFT_ERR_INVALID;
   return mid_needs_filter(mid) ? 1 : 0;
}

int fufft_plan_radices(int64_t n, int variant, int* radices)
{
   const int v = values_per_lane(resolve_variant(n, variant));
   if(!v || !radices || !pow2(n) || n < 2) return FUFFT_ERR_INVALID;
   return factor(n, v, radices);
}

int fufft_plan_chains(int64_t n, int variant, int* chains)
{
   int r[64];
   const int np = fufft_plan_radices(n, variant, r);
   if(np < 0) return np;
   if(!chains) return FUFFT_ERR_INVALID;
   // in-workgroup radix-16 passes use the tap-parity chains, every other pass
   // the single chain (chain_parity / chain_one, fufft_device.hpp)
   for(int i = 0; i < np; i++) chains[i] = r[i] == 16 ? FUFFT_CHAIN_EVENODD : FUFFT_CHAIN_SINGLE;
   return np;
}

int fufft_digit_order(int64_t n, int variant, int32_t* perm)
{
   int r[64];
   const int np = fufft_plan_radices(n, variant, r);
   if(np < 0) return np;
   if(!perm || n > ((int64_t)1 << 30)) return FUFFT_ERR_INVALID;
   for(int64_t i = 0; i < n; i++) perm[i] = group_reverse((int32_t)i, r, np);
   return FUFFT_OK;
}

int fufft_plan_filter_f32(int64_t n, int variant, int layout, int filter_kind,
                          int fold_inv_n, const float* in, float* out)
{
   const int v = values_per_lane(resolve_variant(n, variant));
   if(!v || !in || !out || !pow2(n) || n < v) return FUFFT_ERR_INVALID;
   if(!layout1d_ok(layout)) return FUFFT_ERR_INVALID;
   if(filter_kind != FUFFT_FILTER_SPECTRUM && filter_kind != FUFFT_FILTER_TAPS) return FUFFT_ERR_INVALID;
   int r[64];
   const int np = factor(n, v, r);
   const std::vector<double> s = spectrum_of(n, filter_kind, fold_inv_n, in);
   const uint32_t tlog = (uint32_t)ilog2(n / v), vlog = (uint32_t)ilog2(v);
   for(int64_t i = 0; i < n; i++) {
      const int32_t bin = group_reverse((int32_t)i, r, np);
      // digit-order slot i; lane-major pairs move it to lane_position(i), the
      // reference's bperm slot V*L + k to L + k*T
      const int64_t dst = layout == FUFFT_LAYOUT_DR   ? i
                        : layout == FUFFT_LAYOUT_LANE ? (int64_t)lane_position((uint32_t)i, tlog, vlog)
                                                      : (i >> vlog) + ((i & (v - 1)) << tlog);
      out[2 * dst]     = (float)s[2 * bin];
      out[2 * dst + 1] = (float)s[2 * bin + 1];
   }
   return FUFFT_OK;
}

int fufft_twiddle_table_host(int log_max, float* out)
{
   return fufft_twiddle_table_host_source(log_max, FUFFT_TWIDDLES_ACCURATE, out);
}

int fufft_twiddle_table_host_source(int log_max, int source, float* out)
{
   if(!out || log_max < 1 || log_max > FUFFT_TW_LOG_MAX) return FUFFT_ERR_INVALID;
   if(source != FUFFT_TWIDDLES_ACCURATE && source != FUFFT_TWIDDLES_REFERENCE) return FUFFT_ERR_INVALID;
   fill_table(log_max, out, source);
   return FUFFT_OK;
}

// ---- 1D fp32 --------------------------------------------------------------------------

// the C ABI's mid ids are the registered policies' ids
static_assert(FUFFT_MID_MUL == MID_MUL && FUFFT_MID_CONJ == MID_CONJ && FUFFT_MID_NONE == MID_NONE, "mid ids");
static_assert(mid_known(FUFFT_MID_MUL) && mid_known(FUFFT_MID_CONJ) && mid_known(FUFFT_MID_NONE), "mid ids");
static_assert(mid_needs_filter(FUFFT_MID_MUL) && !mid_needs_filter(FUFFT_MID_NONE), "mid filters");
static_assert(FUFFT_LAYOUT_DR == FLT_DR && FUFFT_LAYOUT_LANE == FLT_LANE && FUFFT_LAYOUT_BPERM == FLT_BPERM,
              "filter layout ids");

// wide: the call is the fused conv, which also runs N = 32768 (wide.hip);
// every other 1D call stops at the single-launch kernels' sizes
static int check_1d(int64_t n, int64_t batch, int variant, int mid, int layout, int* v, bool wide = false)
{
   *v = values_per_lane(resolve_variant(n, variant));
   if(!*v) return FUFFT_ERR_INVALID;
   if(!mid_known(mid)) return FUFFT_ERR_INVALID;
   if(!layout1d_ok(layout)) return FUFFT_ERR_INVALID;
   if(batch < 0 || batch > 0xffffffffll) return FUFFT_ERR_INVALID;
   if(!single_supported(n, *v) && !(wide && conv_wide_plan(n, *v))) return FUFFT_ERR_UNSUPPORTED;
   return FUFFT_OK;
}

static int filter_count(int64_t filt_stride, int64_t n, int64_t batch, uint32_t* fcount)
{
   if(filt_stride == 0) { *fcount = 1; return FUFFT_OK; }
   if(filt_stride == n) { *fcount = (uint32_t)(batch > 0 ? batch : 1); return FUFFT_OK; }
   return FUFFT_ERR_INVALID;
}

// The kernels address a per-transform filter or spectrum array with 32-bit
// byte offsets; a launch whose such array exceeds 4 GiB is split into chunks
// of transforms (the per-transform arrays then advance with the chunk).
static int run_conv1d(int kind, int n, int v, const Conv1dParams& p, void* stream)
{
   if(p.ntrans == 0) return FUFFT_OK;
   hipStream_t s = static_cast<hipStream_t>(stream);
   const uint64_t bytes = (uint64_t)n * 8;
   const bool big_f = (uint64_t)p.fcount * bytes > 0xffffffffull;
   const bool big_s = (uint64_t)p.scount * bytes > 0xffffffffull;
   if(!big_f && !big_s) return status_of(launch_conv1d(kind, n, v, lds_layout(), p, s));
   if((big_f && p.fcount != p.ntrans) || (big_s && p.scount != p.ntrans)) return FUFFT_ERR_INVALID;
   const bool real_in  = kind == K_CONV_R2 || kind == K_FWD_R2;
   const bool real_out = kind == K_CONV_R2 || kind == K_APPLY_R2;
   const uint32_t step = (uint32_t)(0xffffffffull / bytes) & ~255u;
   for(uint32_t t0 = 0; t0 < p.ntrans; t0 += step) {
      const uint32_t cnt = p.ntrans - t0 < step ? p.ntrans - t0 : step;
      const size_t pts = (size_t)t0 * n;
      Conv1dParams q = p;
      q.ntrans = cnt;
      if(p.in0)  q.in0  = static_cast<const char*>(p.in0) + pts * (real_in ? 4 : 8);
      if(p.in1)  q.in1  = static_cast<const char*>(p.in1) + pts * 4;
      if(p.out0) q.out0 = static_cast<char*>(p.out0) + pts * (real_out ? 4 : 8);
      if(p.out1) q.out1 = static_cast<char*>(p.out1) + pts * 4;
      if(p.fcount == p.ntrans && p.filt) { q.filt = static_cast<const char*>(p.filt) + pts * 8; q.fcount = cnt; }
      if(p.scount == p.ntrans && p.spec) { q.spec = static_cast<const char*>(p.spec) + pts * 8; q.scount = cnt; }
      const hipError_t e = launch_conv1d(kind, n, v, lds_layout(), q, s);
      if(e != hipSuccess) return status_of(e);
   }
   return FUFFT_OK;
}

int fufft_conv_f32(const void* in, const void* filt, int64_t filt_stride,
                   void* out, int64_t n, int64_t batch, int mid, int variant,
                   int layout, void* stream)
{
   int v = 0;
   int st = check_1d(n, batch, variant, mid, layout, &v, true);
   if(st != FUFFT_OK) return st;
   if(!in || !out || (mid_needs_filter(mid) && !filt)) return FUFFT_ERR_INVALID;
   if(!aligned16(in) || !aligned16(out) || (filt && !aligned16(filt))) return FUFFT_ERR_ALIGN;
   Conv1dParams p{};
   if((st = filter_count(filt_stride, n, batch, &p.fcount)) != FUFFT_OK) return st;
   const Span si{in, (uint64_t)(n * batch * 8)}, so{out, si.bytes};
   const Span sf{mid_needs_filter(mid) ? filt : nullptr, per_item_bytes(filt_stride, batch, n * 8)};
   if(!same_or_disjoint(si, so) || !disjoint(so, sf)) return FUFFT_ERR_INVALID;
   if((st = current_table(&p.tw)) != FUFFT_OK) return st;
   p.in0 = in; p.filt = filt; p.out0 = out;
   p.ntrans = (uint32_t)batch; p.scount = 1; p.mid = mid; p.fl = layout;
   // N = 32768: one workgroup per transform, 32 values per lane; N = 16384 too
   // for a shared lane-major filter
   if(conv_wide_plan(n, v) ||
      (conv_wide_shared_lane_plan(n, v) && mid_needs_filter(mid) && filt_stride == 0 && layout == FUFFT_LAYOUT_LANE))
      return status_of(launch_conv_wide(p, (int)n, static_cast<hipStream_t>(stream)));
   // one filter per signal at radix 16: the kernels that load each signal's
   // filter with the signal (K_CONV_PSF lane-major, N = 1024 .. 4096;
   // K_CONV_PSF_DR the reference's digit order, N = 2048 .. 4096)
   // (the opt-in XOR LDS layout, a comparison knob, runs the plain kernel)
   const bool per_signal = filt_stride == n && mid_needs_filter(mid) && lds_layout() != LAYOUT_XOR;
   const int kind = per_signal && layout == FUFFT_LAYOUT_LANE &&
                    (conv_psf_plan((int)n, v) || conv_psf_late_plan((int)n, v))             ? K_CONV_PSF
                  : per_signal && layout == FUFFT_LAYOUT_DR && conv_psf_dr_plan((int)n, v) ? K_CONV_PSF_DR
                                                                                           : K_CONV;
   return run_conv1d(kind, (int)n, v, p, stream);
}

static_assert(TIMER_STRIDE == FUFFT_TIMER_STRIDE, "timer record layout");

int fufft_transforms_per_workgroup(int64_t n, int variant)
{
   const int v = values_per_lane(resolve_variant(n, variant));
   if(!v || !fufft_supported(n, variant)) return FUFFT_ERR_UNSUPPORTED;
   const int64_t T = n / v;
   return T >= 128 ? 1 : (int)(256 / T);
}

int fufft_conv_timed_f32(const void* in, const void* filt, int64_t filt_stride, void* out,
                         int64_t n, int64_t batch, int mid, int variant, int layout,
                         uint32_t* timing, int64_t timing_groups, void* stream)
{
   int v = 0;
   int st = check_1d(n, batch, variant, mid, layout, &v);
   if(st != FUFFT_OK) return st;
   if(!in || !out || (mid_needs_filter(mid) && !filt)) return FUFFT_ERR_INVALID;
   if(timing_groups < 0 || timing_groups > 0xffffffffll || (timing_groups > 0 && !timing))
      return FUFFT_ERR_INVALID;
   if(!aligned16(in) || !aligned16(out) || (filt && !aligned16(filt)) || !aligned4(timing))
      return FUFFT_ERR_ALIGN;
   // one launch only, so record g is workgroup g of the whole call
   if(lds_layout() != LAYOUT_DEFAULT) return FUFFT_ERR_UNSUPPORTED;
   Conv1dParams p{};
   if((st = filter_count(filt_stride, n, batch, &p.fcount)) != FUFFT_OK) return st;
   if((uint64_t)p.fcount * (uint64_t)n * 8 > 0xffffffffull) return FUFFT_ERR_UNSUPPORTED;
   const Span si{in, (uint64_t)(n * batch * 8)}, so{out, si.bytes};
   const Span sf{mid_needs_filter(mid) ? filt : nullptr, per_item_bytes(filt_stride, batch, n * 8)};
   const Span st_{timing, (uint64_t)timing_groups * TIMER_STRIDE * 4};
   if(!same_or_disjoint(si, so) || !disjoint(so, sf) || !disjoint(st_, si) || !disjoint(st_, so) ||
      !disjoint(st_, sf))
      return FUFFT_ERR_INVALID;
   if((st = current_table(&p.tw)) != FUFFT_OK) return st;
   p.in0 = in; p.filt = filt; p.out0 = out;
   p.ntrans = (uint32_t)batch; p.scount = 1; p.mid = mid; p.fl = layout;
   p.timing = timing; p.timing_groups = (uint32_t)timing_groups;
   return run_conv1d(K_CONV_TIMED, (int)n, v, p, stream);
}

int fufft_fwd_f32(const void* in, void* spec, int64_t n, int64_t batch,
                  int variant, void* stream)
{
   int v = 0;
   int st = check_1d(n, batch, variant, FUFFT_MID_NONE, FUFFT_LAYOUT_DR, &v);
   if(st != FUFFT_OK) return st;
   if(!in || !spec) return FUFFT_ERR_INVALID;
   if(!aligned16(in) || !aligned16(spec)) return FUFFT_ERR_ALIGN;
   if(!same_or_disjoint({in, (uint64_t)(n * batch * 8)}, {spec, (uint64_t)(n * batch * 8)}))
      return FUFFT_ERR_INVALID;
   Conv1dParams p{};
   if((st = current_table(&p.tw)) != FUFFT_OK) return st;
   p.in0 = in; p.out0 = spec; p.ntrans = (uint32_t)batch;
   p.fcount = 1; p.scount = 1; p.mid = FUFFT_MID_NONE; p.fl = FUFFT_LAYOUT_DR;
   return run_conv1d(K_FWD, (int)n, v, p, stream);
}

int fufft_apply_f32(const void* spec, int64_t spec_stride, const void* filt,
                    int64_t filt_stride, void* out, int64_t n, int64_t batch,
                    int mid, int variant, int layout, void* stream)
{
   int v = 0;
   int st = check_1d(n, batch, variant, mid, layout, &v);
   if(st != FUFFT_OK) return st;
   if(!spec || !out || (mid_needs_filter(mid) && !filt)) return FUFFT_ERR_INVALID;
   if(!aligned16(spec) || !aligned16(out) || (filt && !aligned16(filt))) return FUFFT_ERR_ALIGN;
   Conv1dParams p{};
   if((st = filter_count(filt_stride, n, batch, &p.fcount)) != FUFFT_OK) return st;
   if((st = filter_count(spec_stride, n, batch, &p.scount)) != FUFFT_OK) return st;
   // in place only with one spectrum per transform: a spectrum shared by the
   // batch would be overwritten by the first transform while the others
   // still read it
   const Span ss{spec, per_item_bytes(spec_stride, batch, n * 8)}, so{out, (uint64_t)(n * batch * 8)};
   const Span sf{mid_needs_filter(mid) ? filt : nullptr, per_item_bytes(filt_stride, batch, n * 8)};
   if(!same_or_disjoint(ss, so) || !disjoint(so, sf)) return FUFFT_ERR_INVALID;
   if((st = current_table(&p.tw)) != FUFFT_OK) return st;
   p.spec = spec; p.filt = filt; p.out0 = out;
   p.ntrans = (uint32_t)batch; p.mid = mid; p.fl = layout;
   return run_conv1d(K_APPLY, (int)n, v, p, stream);
}

int fufft_conv_r2_f32(const float* x, const float* y, const void* filt,
                      int64_t filt_stride, float* u, float* v, int64_t n,
                      int64_t batch, int variant, int layout, void* stream)
{
   int vl = 0;
   int st = check_1d(n, batch, variant, FUFFT_MID_MUL, layout, &vl);
   if(st != FUFFT_OK) return st;
   if(!x || !y || !filt || !u || !v) return FUFFT_ERR_INVALID;
   if(!aligned4(x) || !aligned4(y) || !aligned4(u) || !aligned4(v) || !aligned16(filt))
      return FUFFT_ERR_ALIGN;
   Conv1dParams p{};
   if((st = filter_count(filt_stride, n, batch, &p.fcount)) != FUFFT_OK) return st;
   if(!r2_buffers_ok(x, y, filt, filt_stride, u, v, nullptr, 0, n, batch)) return FUFFT_ERR_INVALID;
   if((st = current_table(&p.tw)) != FUFFT_OK) return st;
   p.in0 = x; p.in1 = y; p.filt = filt; p.out0 = u; p.out1 = v;
   p.ntrans = (uint32_t)batch; p.scount = 1; p.mid = FUFFT_MID_MUL; p.fl = layout;
   return run_conv1d(K_CONV_R2, (int)n, vl, p, stream);
}

// ---- natural-order C2C --------------------------------------------------------------

int fufft_c2c_f32(const void* in, void* out, int64_t n, int64_t batch, int direction,
                  int variant, void* stream)
{
   int v = 0;
   int st = check_1d(n, batch, variant, FUFFT_MID_NONE, FUFFT_LAYOUT_DR, &v);
   if(st != FUFFT_OK) return st;
   if(direction != FUFFT_FORWARD && direction != FUFFT_INVERSE) return FUFFT_ERR_INVALID;
   if(!in || !out) return FUFFT_ERR_INVALID;
   if(!aligned16(in) || !aligned16(out)) return FUFFT_ERR_ALIGN;
   if(!same_or_disjoint({in, (uint64_t)(n * batch * 8)}, {out, (uint64_t)(n * batch * 8)}))
      return FUFFT_ERR_INVALID;
   Conv1dParams p{};
   if((st = current_table(&p.tw)) != FUFFT_OK) return st;
   p.in0 = in; p.out0 = out; p.ntrans = (uint32_t)batch;
   p.fcount = 1; p.scount = 1; p.mid = FUFFT_MID_NONE; p.fl = FUFFT_LAYOUT_DR;
   return run_conv1d(direction == FUFFT_FORWARD ? K_C2C_FWD : K_C2C_INV, (int)n, v, p, stream);
}

// ---- filter planning on the device -------------------------------------------------------

static GatherDigits digits_of(const int* radices, int np)
{
   GatherDigits d{};
   d.np = np;
   for(int i = 0; i < np; i++) {
      int w = 0;
      while((1 << w) < radices[i]) w++;
      d.w[i] = (uint8_t)w;
      d.bits += w;
   }
   return d;
}

static int check_plan_kind(int filter_kind)
{
   if(filter_kind != FUFFT_FILTER_SPECTRUM && filter_kind != FUFFT_FILTER_TAPS) return FUFFT_ERR_INVALID;
   return FUFFT_OK;
}

int fufft_plan_filter_device_f32(const void* in, void* out, int64_t n, int64_t count, int variant,
                                 int layout, int filter_kind, int fold_inv_n, void* stream)
{
   int v = 0;
   // a spectrum is only permuted, so the fused conv's N = 32768 plan takes it
   // too; taps need the forward transform, which exists up to N = 16384
   int st = check_1d(n, count, variant, FUFFT_MID_NONE, layout, &v, filter_kind == FUFFT_FILTER_SPECTRUM);
   if(st != FUFFT_OK) return st;
   if((st = check_plan_kind(filter_kind)) != FUFFT_OK) return st;
   if(!in || !out || (filter_kind == FUFFT_FILTER_SPECTRUM && in == out)) return FUFFT_ERR_INVALID;
   if(!aligned16(in) || !aligned16(out)) return FUFFT_ERR_ALIGN;
   if(!same_or_disjoint({in, (uint64_t)(n * count * 8)}, {out, (uint64_t)(n * count * 8)}))
      return FUFFT_ERR_INVALID;
   const float scale = fold_inv_n ? 1.0f / (float)n : 1.0f;   // a power of two: exact
   if(filter_kind == FUFFT_FILTER_SPECTRUM) {
      int r[64];
      GatherParams g{};
      g.in = static_cast<const float2*>(in); g.out = static_cast<float2*>(out);
      g.total = (uint64_t)count * (uint64_t)n;
      g.lane_v = layout != FUFFT_LAYOUT_DR ? v : 0;
      g.bperm = layout == FUFFT_LAYOUT_BPERM ? 1 : 0;
      g.scale = scale;
      g.dw = digits_of(r, factor(n, v, r));
      return status_of(launch_gather(g, static_cast<hipStream_t>(stream)));
   }
   Conv1dParams p{};
   if((st = current_table(&p.tw)) != FUFFT_OK) return st;
   p.in0 = in; p.out0 = out; p.ntrans = (uint32_t)count;
   p.fcount = 1; p.scount = 1; p.mid = FUFFT_MID_NONE; p.fl = layout; p.scale = scale;
   return run_conv1d(K_PLAN_TAPS, (int)n, v, p, stream);
}

// ---- BFP fused conv ------------------------------------------------------------------

int fufft_conv_bfp16(const void* qin, const int8_t* ein, const void* filt,
                     int64_t filt_stride, void* qout, int8_t* eout, int64_t n,
                     int64_t batch, int64_t block, int mid, int variant, int layout,
                     void* stream)
{
   const int vv = resolve_variant(n, variant);
   const int v = values_per_lane(vv);
   if(!v || !mid_known(mid)) return FUFFT_ERR_INVALID;
   if(!layout1d_ok(layout)) return FUFFT_ERR_INVALID;
   if(batch < 0 || batch > 0xffffffffll) return FUFFT_ERR_INVALID;
   if(!pow2(n) || n > 16384 || !bfp_supported((int)n, v)) return FUFFT_ERR_UNSUPPORTED;
   if(!pow2(block) || block < FUFFT_BFP_BLOCK || block > n) return FUFFT_ERR_INVALID;
   if(!qin || !ein || !qout || !eout || (mid_needs_filter(mid) && !filt)) return FUFFT_ERR_INVALID;
   // exponents are read as aligned dwords through the scalar cache
   if(!aligned4(qin) || !aligned4(qout) || !aligned4(ein) || !aligned4(eout) || (filt && !aligned16(filt)))
      return FUFFT_ERR_ALIGN;
   BfpParams p{};
   int st;
   if((st = filter_count(filt_stride, n, batch, &p.fcount)) != FUFFT_OK) return st;
   {
      const uint64_t qb = (uint64_t)(n * batch * 4), eb = (uint64_t)(batch * (n / block));
      const Span sq{qin, qb}, sqo{qout, qb}, se{ein, eb}, seo{eout, eb};
      const Span sf{mid_needs_filter(mid) ? filt : nullptr, per_item_bytes(filt_stride, batch, n * 8)};
      if(!same_or_disjoint(sq, sqo) || !same_or_disjoint(se, seo) || !disjoint(sq, seo) || !disjoint(se, sqo) ||
         !disjoint(sqo, seo) || !disjoint(sf, sqo) || !disjoint(sf, seo))
         return FUFFT_ERR_INVALID;
   }
   if((st = current_table(&p.tw)) != FUFFT_OK) return st;
   if(batch == 0) return FUFFT_OK;
   p.qin = qin; p.ein = ein; p.filt = filt; p.qout = qout; p.eout = eout;
   p.ntrans = (uint32_t)batch; p.mid = mid; p.fl = layout;
   p.log_block = 0;
   while(((int64_t)1 << p.log_block) < block) p.log_block++;
   hipStream_t s = static_cast<hipStream_t>(stream);
   // per-signal filters beyond 4 GiB: chunks keep the 32-bit filter offsets in range
   const uint64_t fbytes = (uint64_t)n * 8;
   if((uint64_t)p.fcount * fbytes <= 0xffffffffull) return status_of(launch_bfp((int)n, v, lds_layout(), p, s));
   const uint32_t step = (uint32_t)(0xffffffffull / fbytes) & ~255u;
   for(uint32_t t0 = 0; t0 < p.ntrans; t0 += step) {
      BfpParams q = p;
      q.ntrans = p.ntrans - t0 < step ? p.ntrans - t0 : step;
      q.fcount = q.ntrans;
      q.qin  = static_cast<const char*>(p.qin) + (size_t)t0 * n * 4;
      q.qout = static_cast<char*>(p.qout) + (size_t)t0 * n * 4;
      q.ein  = p.ein + (size_t)t0 * (n / block);
      q.eout = p.eout + (size_t)t0 * (n / block);
      q.filt = static_cast<const char*>(p.filt) + (size_t)t0 * fbytes;
      const hipError_t e = launch_bfp((int)n, v, lds_layout(), q, s);
      if(e != hipSuccess) return status_of(e);
   }
   return FUFFT_OK;
}

int fufft_conv_bfp16_scaled(const void* qin, const float* sin, const void* qfilt, const float* sfilt,
                            int64_t filt_stride, void* qout, float* sout, int64_t n, int64_t batch,
                            int mid, int variant, int layout, void* stream)
{
   const int v = values_per_lane(resolve_variant(n, variant));
   if(!v || !mid_known(mid) || !layout1d_ok(layout)) return FUFFT_ERR_INVALID;
   if(batch < 0 || batch > 0xffffffffll) return FUFFT_ERR_INVALID;
   if(!pow2(n) || n > 16384 || !bfp_scaled_supported((int)n, v)) return FUFFT_ERR_UNSUPPORTED;
   if(!qin || !sin || !qout || !sout || (mid_needs_filter(mid) && (!qfilt || !sfilt))) return FUFFT_ERR_INVALID;
   if(!aligned4(qin) || !aligned4(qout) || !aligned4(sin) || !aligned4(sout) ||
      (mid_needs_filter(mid) && (!aligned16(qfilt) || !aligned4(sfilt))))
      return FUFFT_ERR_ALIGN;
   BfpScaledParams p{};
   int st;
   if((st = filter_count(filt_stride, n, batch, &p.fcount)) != FUFFT_OK) return st;
   {
      const uint64_t qb = (uint64_t)(n * batch * 4), sb = (uint64_t)(batch * 4);
      const Span sq{qin, qb}, sqo{qout, qb}, ss{sin, sb}, sso{sout, sb};
      const bool f = mid_needs_filter(mid);
      const Span sqf{f ? qfilt : nullptr, per_item_bytes(filt_stride, batch, n * 4)};
      const Span ssf{f ? sfilt : nullptr, per_item_bytes(filt_stride, batch, 4)};
      if(!same_or_disjoint(sq, sqo) || !same_or_disjoint(ss, sso) || !disjoint(sq, sso) || !disjoint(ss, sqo) ||
         !disjoint(sqo, sso) || !disjoint(sqf, sqo) || !disjoint(sqf, sso) || !disjoint(ssf, sqo) ||
         !disjoint(ssf, sso))
         return FUFFT_ERR_INVALID;
   }
   if((st = current_table(&p.tw)) != FUFFT_OK) return st;
   if(batch == 0) return FUFFT_OK;
   p.qin = qin; p.sin = sin; p.qfilt = qfilt; p.sfilt = sfilt; p.qout = qout; p.sout = sout;
   p.ntrans = (uint32_t)batch; p.mid = mid; p.fl = layout;
   hipStream_t s = static_cast<hipStream_t>(stream);
   // per-signal filters beyond 4 GiB: chunks keep the 32-bit filter offsets in range
   const uint64_t fbytes = (uint64_t)n * 4;
   if((uint64_t)p.fcount * fbytes <= 0xffffffffull) return status_of(launch_bfp_scaled((int)n, v, p, s));
   const uint32_t step = (uint32_t)(0xffffffffull / fbytes) & ~255u;
   for(uint32_t t0 = 0; t0 < p.ntrans; t0 += step) {
      BfpScaledParams q = p;
      q.ntrans = p.ntrans - t0 < step ? p.ntrans - t0 : step;
      q.fcount = q.ntrans;
      q.qin   = static_cast<const char*>(p.qin) + (size_t)t0 * n * 4;
      q.qout  = static_cast<char*>(p.qout) + (size_t)t0 * n * 4;
      q.sin   = p.sin + t0;
      q.sout  = p.sout + t0;
      q.qfilt = static_cast<const char*>(p.qfilt) + (size_t)t0 * fbytes;
      q.sfilt = p.sfilt + t0;
      const hipError_t e = launch_bfp_scaled((int)n, v, q, s);
      if(e != hipSuccess) return status_of(e);
   }
   return FUFFT_OK;
}

// ---- HBM stream ceiling --------------------------------------------------------------

int fufft_stream_f32(const void* in, void* out, int64_t bytes, int nontemporal, void* stream)
{
   if(!in || !out || in == out || bytes < 0 || (bytes & 15) || (nontemporal != 0 && nontemporal != 1))
      return FUFFT_ERR_INVALID;
   if(!aligned16(in) || !aligned16(out)) return FUFFT_ERR_ALIGN;
   if(!disjoint({in, (uint64_t)bytes}, {out, (uint64_t)bytes})) return FUFFT_ERR_INVALID;
   return status_of(launch_stream(in, out, (uint64_t)bytes, nontemporal != 0, static_cast<hipStream_t>(stream)));
}

int fufft_stream_shape_f32(const void* in, void* out, int64_t bytes, int lanes, int load_bytes,
                           int loads_per_lane, int tiles_per_group, int groups, int load_policy,
                           int store_policy, void* stream)
{
   if(!in || !out || in == out || bytes < 0 || (bytes & 15)) return FUFFT_ERR_INVALID;
   if(!stream_shape_ok(lanes, load_bytes, loads_per_lane, tiles_per_group, groups, load_policy, store_policy))
      return FUFFT_ERR_INVALID;
   if(!aligned16(in) || !aligned16(out)) return FUFFT_ERR_ALIGN;
   if(!disjoint({in, (uint64_t)bytes}, {out, (uint64_t)bytes})) return FUFFT_ERR_INVALID;
   return status_of(launch_stream_shape(in, out, (uint64_t)bytes, lanes, load_bytes, loads_per_lane,
                                        tiles_per_group, groups, load_policy, store_policy,
                                        static_cast<hipStream_t>(stream)));
}

// ---- BFP host codec -----------------------------------------------------------------

int fufft_bfp_exponent(float absmax)
{
   uint32_t bits;
   std::memcpy(&bits, &absmax, sizeof bits);
   bits &= 0x7fffffffu;
   const uint32_t xb = bits >> 23;
   if(xb == 0) return -128;
   // absmax = m * 2^(xb-126), m in [0.5, 1); 32767 * 2^(xb-141) >= absmax
   // exactly when the 23 fraction bits are <= 0x7ffe00
   const int e = (int)xb - 141 + ((bits & 0x7fffffu) > 0x7ffe00u ? 1 : 0);
   return e < -128 ? -128 : e;
}

int fufft_bfp_quantize(const float* x, int64_t npts, int64_t block, int16_t* q, int8_t* e)
{
   if(!x || !q || !e || npts < 0 || block < 1 || npts % block) return FUFFT_ERR_INVALID;
   for(int64_t b = 0; b < npts / block; b++) {
      const float* xb = x + 2 * b * block;
      float m = 0.0f;
      for(int64_t i = 0; i < 2 * block; i++) m = std::fmax(m, std::fabs(xb[i]));
      const int ex = fufft_bfp_exponent(m);
      e[b] = (int8_t)ex;
      for(int64_t i = 0; i < 2 * block; i++)
         q[2 * b * block + i] = (int16_t)std::rint(std::ldexp(xb[i], -ex));
   }
   return FUFFT_OK;
}

int fufft_bfp_dequantize(const int16_t* q, const int8_t* e, int64_t npts, int64_t block, float* x)
{
   if(!x || !q || !e || npts < 0 || block < 1 || npts % block) return FUFFT_ERR_INVALID;
   for(int64_t b = 0; b < npts / block; b++)
      for(int64_t i = 0; i < 2 * block; i++)
         x[2 * b * block + i] = std::ldexp((float)q[2 * b * block + i], e[b]);
   return FUFFT_OK;
}

// The reference's rule, verify_kernel.cpp:1092-1105 (bfp_quantize): per
// transform of n points, mx = max(abs-max of the re and im parts, 1e-30),
// q = rint(clamp(x * (32767 / mx), -32767, 32767)), scale = mx / 32767.
int fufft_bfp_scaled_quantize(const float* x, int64_t n, int64_t count, int16_t* q, float* scale)
{
   if(!x || !q || !scale || n < 1 || count < 0) return FUFFT_ERR_INVALID;
   for(int64_t t = 0; t < count; t++) {
      const float* xt = x + 2 * t * n;
      float mx = 0.0f;
      for(int64_t i = 0; i < 2 * n; i++) mx = std::max(mx, std::fabs(xt[i]));
      mx = std::max(mx, 1e-30f);
      const float inv = 32767.0f / mx;
      for(int64_t i = 0; i < 2 * n; i++)
         q[2 * t * n + i] = (int16_t)std::lrint(std::min(std::max(xt[i] * inv, -32767.0f), 32767.0f));
      scale[t] = mx / 32767.0f;
   }
   return FUFFT_OK;
}

int fufft_bfp_scaled_dequantize(const int16_t* q, const float* scale, int64_t n, int64_t count, float* x)
{
   if(!x || !q || !scale || n < 1 || count < 0) return FUFFT_ERR_INVALID;
   for(int64_t t = 0; t < count; t++)
      for(int64_t i = 0; i < 2 * n; i++) x[2 * t * n + i] = (float)q[2 * t * n + i] * scale[t];
   return FUFFT_OK;
}

// ---- four-step large N -----------------------------------------------------------------

int fufft_large_plan(int64_t n, int* lout, int* mid)
{
   if(!lout || !mid) return FUFFT_ERR_INVALID;
   if(!pow2(n) || n < 8192 || n > ((int64_t)1 << FUFFT_TW_LOG_MAX)) return FUFFT_ERR_UNSUPPORTED;
   // fewest outer levels that bring the middle to a single-workgroup size
   // <= 4096; the middle then lies in [512, 4096], which both middles (radix
   // 16 and radix 8) cover
   int lo = 1;
   while((n >> (4 * lo)) > 4096) lo++;
   *lout = lo;
   *mid = (int)(n >> (4 * lo));
   return FUFFT_OK;
}

// chain radices: lout radix-16 outer levels, then the middle's own plan at
// v values per lane -- the order of bench_fufft.cu:410-428
static int large_radices(int64_t n, int v, int* lout, int* mid, int* r)
{
   if(!v) return FUFFT_ERR_INVALID;
   const int st = fufft_large_plan(n, lout, mid);
   if(st != FUFFT_OK) return st;
   int np = 0;
   for(int i = 0; i < *lout; i++) r[np++] = 16;
   np += factor(*mid, v, r + np);
   return np;
}

int fufft_large_digit_order(int64_t n, int variant, int32_t* perm)
{
   int r[64], lout = 0, mid = 0;
   const int np = large_radices(n, large_middle_v(variant), &lout, &mid, r);
   if(np < 0) return np;
   if(!perm) return FUFFT_ERR_INVALID;
   for(int64_t i = 0; i < n; i++) perm[i] = group_reverse((int32_t)i, r, np);
   return FUFFT_OK;
}

int fufft_plan_filter_large_f32(int64_t n, int variant, int filter_kind, int fold_inv_n, const float* in,
                                float* out)
{
   int r[64], lout = 0, mid = 0;
   const int np = large_radices(n, large_middle_v(variant), &lout, &mid, r);
   if(np < 0) return np;
   if(!in || !out) return FUFFT_ERR_INVALID;
   if(filter_kind != FUFFT_FILTER_SPECTRUM && filter_kind != FUFFT_FILTER_TAPS) return FUFFT_ERR_INVALID;
   const std::vector<double> s = spectrum_of(n, filter_kind, fold_inv_n, in);
   for(int64_t i = 0; i < n; i++) {
      const int32_t bin = group_reverse((int32_t)i, r, np);
      out[2 * i]     = (float)s[2 * bin];
      out[2 * i + 1] = (float)s[2 * bin + 1];
   }
   return FUFFT_OK;
}

// the forward (DIF, largest stride first) or inverse (DIT, smallest first)
// outer levels of a four-step plan; two levels run as one fused pass
static hipError_t outer_levels(float2* a, int64_t n, int64_t batch, int lout, bool dit, const float2* tw,
                               hipStream_t s)
{
   if(lout == 2) return launch_outer2_pass(a, n, batch, dit, tw, s);
   hipError_t e = hipSuccess;
   for(int i = 0; i < lout && e == hipSuccess; i++) {
      const int l = dit ? lout - 1 - i : i;
      e = launch_outer_pass(a, n, batch, n >> (4 * (l + 1)), dit, tw, s);
   }
   return e;
}

int fufft_plan_filter_large_device_f32(const void* in, void* out, int64_t n, int64_t count,
                                       int variant, int filter_kind, int fold_inv_n, void* stream)
{
   int r[64], lout = 0, mn = 0;
   const int v = large_middle_v(variant);
   const int np = large_radices(n, v, &lout, &mn, r);
   if(np < 0) return np;
   int st = check_plan_kind(filter_kind);
   if(st != FUFFT_OK) return st;
   if(count < 0 || count * (n / 16) > 0xffffffffll) return FUFFT_ERR_INVALID;
   if(!in || !out || (filter_kind == FUFFT_FILTER_SPECTRUM && in == out)) return FUFFT_ERR_INVALID;
   if(!aligned16(in) || !aligned16(out)) return FUFFT_ERR_ALIGN;
   if(!same_or_disjoint({in, (uint64_t)(n * count * 8)}, {out, (uint64_t)(n * count * 8)}))
      return FUFFT_ERR_INVALID;
   const float2* tw = nullptr;
   if((st = current_table(&tw)) != FUFFT_OK) return st;
   if(count == 0) return FUFFT_OK;
   hipStream_t s = static_cast<hipStream_t>(stream);
   const float scale = fold_inv_n ? 1.0f / (float)n : 1.0f;
   if(filter_kind == FUFFT_FILTER_SPECTRUM) {
      GatherParams g{};
      g.in = static_cast<const float2*>(in); g.out = static_cast<float2*>(out);
      g.total = (uint64_t)count * (uint64_t)n;
      g.scale = scale;
      g.dw = digits_of(r, np);
      return status_of(launch_gather(g, s));
   }
   // taps: the forward half of the four-step chain, in place on out
   if(in != out && hipMemcpyAsync(out, in, (size_t)count * n * 8, hipMemcpyDeviceToDevice, s) != hipSuccess)
      return FUFFT_ERR_HIP;
   if(const hipError_t e = outer_levels(static_cast<float2*>(out), n, count, lout, false, tw, s); e != hipSuccess)
      return status_of(e);
   Conv1dParams p{};
   p.tw = tw; p.in0 = out; p.out0 = out;
   p.ntrans = (uint32_t)(count * (n / mn));
   p.fcount = 1; p.scount = 1; p.mid = FUFFT_MID_NONE; p.fl = FUFFT_LAYOUT_DR; p.scale = scale;
   return run_conv1d(K_PLAN_TAPS, mn, v, p, stream);
}

int fufft_conv_large_f32(void* buf, const void* filt, int64_t filt_stride, int64_t n,
                         int64_t batch, int mid, int variant, void* stream)
{
   int lout = 0, mn = 0;
   int st = fufft_large_plan(n, &lout, &mn);
   if(st != FUFFT_OK) return st;
   const int v = large_middle_v(variant);
   if(!mid_known(mid) || !v) return FUFFT_ERR_INVALID;
   if(batch < 0 || batch * (n / 16) > 0xffffffffll) return FUFFT_ERR_INVALID;
   if(!buf || (mid_needs_filter(mid) && !filt)) return FUFFT_ERR_INVALID;
   if(!aligned16(buf) || (filt && !aligned16(filt))) return FUFFT_ERR_ALIGN;
   if(filt_stride != 0 && filt_stride != n) return FUFFT_ERR_INVALID;
   if(!conv1d_supported(mn, v)) return FUFFT_ERR_UNSUPPORTED;
   if(!disjoint({buf, (uint64_t)(n * batch * 8)},
                {mid_needs_filter(mid) ? filt : nullptr, per_item_bytes(filt_stride, batch, n * 8)}))
      return FUFFT_ERR_INVALID;
   Conv1dParams p{};
   if((st = current_table(&p.tw)) != FUFFT_OK) return st;
   if(batch == 0) return FUFFT_OK;
   hipStream_t s = static_cast<hipStream_t>(stream);
   // The three stages run over sub-batches small enough for the data to stay
   // in the last-level cache from one stage to the next.  One filter per
   // transform streams a sub-batch's worth of filter bytes through the
   // middle as well, so the sub-batch is halved: data and filter slices
   // together fill the cache.  N = 32768, filter per transform, Gpt/s at
   // 64 / 96 / 128 / 192 / 256 MiB: 106.3 / 109.0 / 115.0 / 115.7 / 101.3
   // (a shared filter: 117.1 / 123.5 / 128.6 / 133.3 / 136.8), same box.
   const int64_t sub = subbatch_items(n * 8 * (filt_stride == n && mid_needs_filter(mid) ? 2 : 1), batch,
                                      SUBBATCH_FOURSTEP_MB);
   for(int64_t t0 = 0; t0 < batch; t0 += sub) {
      const int64_t nb = batch - t0 < sub ? batch - t0 : sub;
      float2* a = static_cast<float2*>(buf) + t0 * n;
      // forward outer levels, largest stride first
      hipError_t e = outer_levels(a, n, nb, lout, false, p.tw, s);
      if(e != hipSuccess) return status_of(e);
      // the middle: every mn-point chunk is one fused conv, in place; chunk c
      // of a transform uses filter slots [c*mn, (c+1)*mn) of the chained order
      const int64_t chunks = nb * (n / mn);
      Conv1dParams q = p;
      q.in0 = a; q.out0 = a;
      q.filt = (filt_stride == 0 || !filt) ? filt : static_cast<const char*>(filt) + t0 * n * 8;
      q.ntrans = (uint32_t)chunks;
      q.fcount = (uint32_t)(filt_stride == 0 ? n / mn : chunks);
      q.scount = 1; q.mid = mid; q.fl = FUFFT_LAYOUT_DR;
      if((st = run_conv1d(K_CONV_MID, mn, v, q, stream)) != FUFFT_OK) return st;
      // inverse outer levels, smallest stride first
      e = outer_levels(a, n, nb, lout, true, p.tw, s);
      if(e != hipSuccess) return status_of(e);
   }
   return FUFFT_OK;
}

}  // extern "C"

// ---- 2D ------------------------------------------------------------------------------
// Rows use the 1D kernels (radix 8 at w = 512, 4096, 8192, radix 16 elsewhere);
// columns the column kernels (conv2d.hip).
// Images of at most 8192 points (8 <= h, w <= 512) run the fused small-image
// kernel instead, radix 8 both ways; their column order is the identity, so
// FUFFT_LAYOUT_LANE and FUFFT_LAYOUT_DR name the same filter there.

extern "C" int fufft_plan2d(int64_t h, int64_t w, int* v_rows, int* v_cols)
{
   if(!v_rows || !v_cols) return FUFFT_ERR_INVALID;
   if(small2d_supported(h, w)) {
      *v_rows = 8;
      *v_cols = 8;
      return FUFFT_OK;
   }
   if(!pow2(h) || !pow2(w) || h > 2048 || w > 16384) return FUFFT_ERR_UNSUPPORTED;
   // rows: radix 8 at w = 512, 4096 and 8192, radix 16 elsewhere.  At the
   // powers of 8 this is the reference's own 2D plan (radix 8 both ways,
   // verify_kernel.cpp:700-722), so its 2D results come out bit for bit
   const int vr = (w == 512 || w == 4096 || w == 8192) ? 8 : 16;
   const int vc = col_values_per_lane((int)h);
   if(!vc || !vr || !conv1d_supported((int)w, vr)) return FUFFT_ERR_UNSUPPORTED;
   *v_rows = vr;
   *v_cols = vc;
   return FUFFT_OK;
}

namespace {

struct Plan2d {
   int vr = 0, vc = 0, nr = 0, nc = 0;
   bool small = false;          // the fused small-image kernel
   int rr[64], rc[64];
};

int plan2d(int64_t h, int64_t w, Plan2d* p)
{
   const int st = fufft_plan2d(h, w, &p->vr, &p->vc);
   if(st != FUFFT_OK) return st;
   p->small = small2d_supported(h, w);
   p->nr = factor(w, p->vr, p->rr);
   p->nc = factor(h, p->vc, p->rc);
   return FUFFT_OK;
}

int check_2d(int64_t h, int64_t w, int64_t batch, Plan2d* p)
{
   const int st = plan2d(h, w, p);
   if(st != FUFFT_OK) return st;
   if(batch < 0 || batch * h > 0xffffffffll) return FUFFT_ERR_INVALID;
   return FUFFT_OK;
}

// the three launches of a 2D pass share this row-launch helper: n = w points
// per row, h * batch rows.  Row spectra are lane-major (position c of a row
// holds digit-order slot lane_slot(c)): the row forward then stores and the
// row inverse loads whole contiguous runs per wavefront.  The column kernels
// do not care which slot a column holds, so 2D filters and spectra carry
// their columns in the same order (fufft_plan2d_column_order).
Conv1dParams rows_params(const float2* tw, int64_t h, int64_t batch)
{
   Conv1dParams p{};
   p.tw = tw;
   p.ntrans = (uint32_t)(h * batch);
   p.fcount = 1; p.scount = 1; p.mid = FUFFT_MID_NONE; p.fl = FUFFT_LAYOUT_DR;
   p.sl = FUFFT_LAYOUT_LANE;
   return p;
}

// digit-order slot held by column c of a 2D row spectrum (lane-major rows)
int64_t column_slot(int64_t c, int64_t w, int vr)
{
   return lane_slot((uint32_t)c, (uint32_t)ilog2(w / vr), (uint32_t)ilog2(vr));
}

// the same for a plan: the identity for small images
int64_t column_slot(const Plan2d& pl, int64_t c, int64_t w)
{
   return pl.small ? c : column_slot(c, w, pl.vr);
}

ColParams col_params(const float2* tw, int64_t w, int64_t batch)
{
   ColParams c{};
   c.tw = tw; c.nimg = (uint32_t)batch; c.fcount = 1; c.scount = 1; c.mid = FUFFT_MID_NONE;
   c.w = (uint32_t)w;
   return c;
}

// the column kernels' filter read for a 2D filter in `layout`: FUFFT_LAYOUT_LANE
// is the row spectra's own column order; FUFFT_LAYOUT_DR is the reference's,
// read through the column -> slot map
void set_filter_layout(ColParams& c, const Plan2d& pl, int64_t w, int layout)
{
   c.f_dr = layout == FUFFT_LAYOUT_DR ? 1u : 0u;
   c.f_tr_log = (uint32_t)ilog2(w / pl.vr);
   c.f_vr_log = (uint32_t)ilog2(pl.vr);
}

bool layout_ok(int layout) { return layout == FUFFT_LAYOUT_DR || layout == FUFFT_LAYOUT_LANE; }

// The two-for-one 2D conv in sub-batches of `sub` images.  The packed complex
// images of sub-batch i0 go to work + i0 * h * w (a caller workspace of
// batch images), or to the start of work for every sub-batch when reuse_work
// is set (a workspace of sub images; the launches of one stream run in
// order, so a sub-batch's three launches finish before the next reuses it).
int conv2d_r2_run(const Plan2d& pl, const float* x, const float* y, const void* filt,
                  int64_t filt_stride, float* u, float* v, char* work, bool reuse_work, int64_t sub,
                  int64_t h, int64_t w, int64_t batch, int layout, const float2* tw, void* stream)
{
   hipStream_t s = static_cast<hipStream_t>(stream);
   const int64_t np = h * w;
   for(int64_t i0 = 0; i0 < batch; i0 += sub) {
      const int64_t nb = batch - i0 < sub ? batch - i0 : sub;
      char* wk = reuse_work ? work : work + i0 * np * 8;
      // z = x + i y: rows DIF straight from the two real arrays into work
      Conv1dParams r = rows_params(tw, h, nb);
      r.in0 = x + i0 * np; r.in1 = y + i0 * np; r.out0 = wk;
      int st = run_conv1d(K_FWD_R2, (int)w, pl.vr, r, stream);
      if(st != FUFFT_OK) return st;
      ColParams c = col_params(tw, w, nb);
      set_filter_layout(c, pl, w, layout);
      c.in = wk; c.out = wk; c.mid = FUFFT_MID_MUL;
      c.filt = filt_stride == 0 ? filt : static_cast<const char*>(filt) + i0 * np * 8;
      c.fcount = (uint32_t)(filt_stride == 0 ? 1 : nb);
      const hipError_t e = launch_col(COL_CONV, (int)h, c, s);
      if(e != hipSuccess) return status_of(e);
      // rows DIT from work; Re -> u, Im -> v (a real filter keeps them apart)
      r = rows_params(tw, h, nb);
      r.spec = wk; r.scount = r.ntrans; r.out0 = u + i0 * np; r.out1 = v + i0 * np;
      if((st = run_conv1d(K_APPLY_R2, (int)w, pl.vr, r, stream)) != FUFFT_OK) return st;
   }
   return FUFFT_OK;
}

}  // namespace

extern "C" {

int fufft_plan2d_column_order(int64_t h, int64_t w, int32_t* slot)
{
   Plan2d pl;
   const int st = plan2d(h, w, &pl);
   if(st != FUFFT_OK) return st;
   if(!slot) return FUFFT_ERR_INVALID;
   for(int64_t c = 0; c < w; c++) slot[c] = (int32_t)column_slot(pl, c, w);
   return FUFFT_OK;
}

int fufft_plan_filter2d_f32(int64_t h, int64_t w, int layout, int filter_kind, int fold_inv_n,
                            const float* in, float* out)
{
   Plan2d pl;
   int st = plan2d(h, w, &pl);
   if(st != FUFFT_OK) return st;
   if(!in || !out || !layout_ok(layout)) return FUFFT_ERR_INVALID;
   if(filter_kind != FUFFT_FILTER_SPECTRUM && filter_kind != FUFFT_FILTER_TAPS) return FUFFT_ERR_INVALID;
   const int64_t np = h * w;
   std::vector<double> s(2 * (size_t)np);
   for(int64_t i = 0; i < 2 * np; i++) s[i] = in[i];
   if(filter_kind == FUFFT_FILTER_TAPS) {
      std::vector<double> line(2 * (size_t)(h > w ? h : w));
      for(int64_t r = 0; r < h; r++) {
         line.assign(s.begin() + 2 * r * w, s.begin() + 2 * (r + 1) * w);
         dft_f64(line, w, -1);
         std::copy(line.begin(), line.begin() + 2 * w, s.begin() + 2 * r * w);
      }
      line.resize(2 * (size_t)h);
      for(int64_t c = 0; c < w; c++) {
         for(int64_t r = 0; r < h; r++) { line[2 * r] = s[2 * (r * w + c)]; line[2 * r + 1] = s[2 * (r * w + c) + 1]; }
         dft_f64(line, h, -1);
         for(int64_t r = 0; r < h; r++) { s[2 * (r * w + c)] = line[2 * r]; s[2 * (r * w + c) + 1] = line[2 * r + 1]; }
      }
   }
   const double scale = fold_inv_n ? 1.0 / (double)np : 1.0;
   for(int64_t r = 0; r < h; r++) {
      const int64_t br = group_reverse((int32_t)r, pl.rc, pl.nc);
      for(int64_t c = 0; c < w; c++) {
         const int64_t sc = layout == FUFFT_LAYOUT_LANE ? column_slot(pl, c, w) : c;
         const int64_t bc = group_reverse((int32_t)sc, pl.rr, pl.nr);
         out[2 * (r * w + c)]     = (float)(s[2 * (br * w + bc)] * scale);
         out[2 * (r * w + c) + 1] = (float)(s[2 * (br * w + bc) + 1] * scale);
      }
   }
   return FUFFT_OK;
}

int fufft_plan_filter2d_device_f32(const void* in, void* out, int64_t h, int64_t w, int64_t count,
                                   int layout, int filter_kind, int fold_inv_n, void* stream)
{
   Plan2d pl;
   int st = check_2d(h, w, count, &pl);
   if(st != FUFFT_OK) return st;
   if((st = check_plan_kind(filter_kind)) != FUFFT_OK) return st;
   if(!layout_ok(layout)) return FUFFT_ERR_INVALID;
   if(!in || !out || (filter_kind == FUFFT_FILTER_SPECTRUM && in == out)) return FUFFT_ERR_INVALID;
   if(!aligned16(in) || !aligned16(out)) return FUFFT_ERR_ALIGN;
   if(!same_or_disjoint({in, (uint64_t)(h * w * count * 8)}, {out, (uint64_t)(h * w * count * 8)}))
      return FUFFT_ERR_INVALID;
   const float2* tw = nullptr;
   if((st = current_table(&tw)) != FUFFT_OK) return st;
   if(count == 0) return FUFFT_OK;
   hipStream_t s = static_cast<hipStream_t>(stream);
   const float scale = fold_inv_n ? 1.0f / (float)(h * w) : 1.0f;
   if(filter_kind == FUFFT_FILTER_SPECTRUM) {
      GatherParams g{};
      g.in = static_cast<const float2*>(in); g.out = static_cast<float2*>(out);
      g.total = (uint64_t)count * (uint64_t)(h * w);
      g.scale = scale;
      g.dh = digits_of(pl.rc, pl.nc);
      g.dw = digits_of(pl.rr, pl.nr);
      g.lane_v = (layout == FUFFT_LAYOUT_LANE && !pl.small) ? pl.vr : 0;
      return status_of(launch_gather(g, s));
   }
   // taps of a small image: plan them on the host (fufft_plan_filter2d_f32)
   if(pl.small) return FUFFT_ERR_UNSUPPORTED;
   // taps: rows DIF (scaled) into out, then columns DIF in place -- the
   // forward half of fufft_conv2d_f32
   Conv1dParams r = rows_params(tw, h, count);
   r.in0 = in; r.out0 = out; r.scale = scale; r.fl = layout;
   if((st = run_conv1d(K_PLAN_TAPS, (int)w, pl.vr, r, stream)) != FUFFT_OK) return st;
   ColParams c = col_params(tw, w, count);
   c.in = out; c.out = out;
   return status_of(launch_col(COL_FWD, (int)h, c, s));
}

int fufft_conv2d_f32(const void* in, const void* filt, int64_t filt_stride, void* out,
                     int64_t h, int64_t w, int64_t batch, int mid, int layout, void* stream)
{
   Plan2d pl;
   int st = check_2d(h, w, batch, &pl);
   if(st != FUFFT_OK) return st;
   if(!mid_known(mid) || !layout_ok(layout)) return FUFFT_ERR_INVALID;
   if(!in || !out || (mid_needs_filter(mid) && !filt)) return FUFFT_ERR_INVALID;
   if(!aligned16(in) || !aligned16(out) || (filt && !aligned16(filt))) return FUFFT_ERR_ALIGN;
   if(filt_stride != 0 && filt_stride != h * w) return FUFFT_ERR_INVALID;
   {
      const Span si{in, (uint64_t)(h * w * batch * 8)}, so{out, si.bytes};
      const Span sf{mid_needs_filter(mid) ? filt : nullptr, per_item_bytes(filt_stride, batch, h * w * 8)};
      if(!same_or_disjoint(si, so) || !disjoint(so, sf)) return FUFFT_ERR_INVALID;
   }
   const float2* tw = nullptr;
   if((st = current_table(&tw)) != FUFFT_OK) return st;
   if(batch == 0) return FUFFT_OK;
   hipStream_t s = static_cast<hipStream_t>(stream);
   if(pl.small) {
      Small2dParams q{};
      q.in = in; q.out = out; q.filt = filt; q.tw = tw; q.mid = mid;
      q.nimg = (uint32_t)batch;
      q.fcount = (uint32_t)(filt_stride == 0 ? 1 : batch);
      return status_of(launch_small2d((int)h, (int)w, q, s));
   }
   const int64_t np = h * w, sub = subbatch_items(np * 8, batch, SUBBATCH_2D_MB);
   for(int64_t i0 = 0; i0 < batch; i0 += sub) {
      const int64_t nb = batch - i0 < sub ? batch - i0 : sub;
      const char* src = static_cast<const char*>(in) + i0 * np * 8;
      char* dst = static_cast<char*>(out) + i0 * np * 8;
      // rows DIF into digit order (out), columns DIF -> mid -> DIT in place,
      // rows DIT in place
      Conv1dParams r = rows_params(tw, h, nb);
      r.in0 = src; r.out0 = dst;
      if((st = run_conv1d(K_FWD, (int)w, pl.vr, r, stream)) != FUFFT_OK) return st;
      ColParams c = col_params(tw, w, nb);
      set_filter_layout(c, pl, w, layout);
      c.in = dst; c.out = dst; c.mid = mid;
      c.filt = (filt_stride == 0 || !filt) ? filt : static_cast<const char*>(filt) + i0 * np * 8;
      c.fcount = (uint32_t)(filt_stride == 0 ? 1 : nb);
      const hipError_t e = launch_col(COL_CONV, (int)h, c, s);
      if(e != hipSuccess) return status_of(e);
      r = rows_params(tw, h, nb);
      r.spec = dst; r.scount = r.ntrans; r.out0 = dst;
      if((st = run_conv1d(K_APPLY, (int)w, pl.vr, r, stream)) != FUFFT_OK) return st;
   }
   return FUFFT_OK;
}

int fufft_conv2d_r2_f32(const float* x, const float* y, const void* filt, int64_t filt_stride,
                        float* u, float* v, void* work, int64_t h, int64_t w, int64_t batch,
                        int layout, void* stream)
{
   Plan2d pl;
   int st = check_2d(h, w, batch, &pl);
   if(st != FUFFT_OK) return st;
   if(pl.small) return FUFFT_ERR_UNSUPPORTED;      // the fused conv only, as in the reference
   if(!x || !y || !filt || !u || !v || !work || !layout_ok(layout)) return FUFFT_ERR_INVALID;
   if(!aligned4(x) || !aligned4(y) || !aligned4(u) || !aligned4(v) || !aligned16(filt) ||
      !aligned16(work))
      return FUFFT_ERR_ALIGN;
   if(filt_stride != 0 && filt_stride != h * w) return FUFFT_ERR_INVALID;
   if(!r2_buffers_ok(x, y, filt, filt_stride, u, v, work, (uint64_t)(h * w * batch * 8), h * w, batch))
      return FUFFT_ERR_INVALID;
   const float2* tw = nullptr;
   if((st = current_table(&tw)) != FUFFT_OK) return st;
   const int64_t sub = subbatch_items(h * w * 8, batch, SUBBATCH_2D_MB);
   return conv2d_r2_run(pl, x, y, filt, filt_stride, u, v, static_cast<char*>(work), false, sub, h, w,
                        batch, layout, tw, stream);
}

int fufft_conv2d_r2_noalloc_f32(const float* x, const float* y, const void* filt, int64_t filt_stride,
                                float* u, float* v, int64_t h, int64_t w, int64_t batch, int layout,
                                void* stream)
{
   Plan2d pl;
   int st = check_2d(h, w, batch, &pl);
   if(st != FUFFT_OK) return st;
   if(pl.small) return FUFFT_ERR_UNSUPPORTED;      // the fused conv only, as in the reference
   if(!x || !y || !filt || !u || !v || !layout_ok(layout)) return FUFFT_ERR_INVALID;
   if(!aligned4(x) || !aligned4(y) || !aligned4(u) || !aligned4(v) || !aligned16(filt)) return FUFFT_ERR_ALIGN;
   if(filt_stride != 0 && filt_stride != h * w) return FUFFT_ERR_INVALID;
   const int64_t img_bytes = h * w * 8;
   if(img_bytes > FUFFT_SCRATCH_BYTES) return FUFFT_ERR_SCRATCH;
   if(!r2_buffers_ok(x, y, filt, filt_stride, u, v, nullptr, 0, h * w, batch)) return FUFFT_ERR_INVALID;
   const float2* tw = nullptr;
   float2* scr = nullptr;
   if((st = current_table(&tw, &scr)) != FUFFT_OK) return st;
   // the usual sub-batch, capped at what the scratch holds; every sub-batch
   // reuses the scratch from its start (the row forward writes all of it
   // before the column and row-inverse launches read it)
   int64_t sub = subbatch_items(img_bytes, batch, SUBBATCH_2D_MB);
   const int64_t cap = FUFFT_SCRATCH_BYTES / img_bytes;
   if(sub > cap) sub = cap;
   return conv2d_r2_run(pl, x, y, filt, filt_stride, u, v, reinterpret_cast<char*>(scr), true, sub, h, w,
                        batch, layout, tw, stream);
}

int fufft_fwd2d_f32(const void* in, void* spec, int64_t h, int64_t w, int64_t batch, void* stream)
{
   Plan2d pl;
   int st = check_2d(h, w, batch, &pl);
   if(st != FUFFT_OK) return st;
   if(pl.small) return FUFFT_ERR_UNSUPPORTED;      // the fused conv only, as in the reference
   if(!in || !spec) return FUFFT_ERR_INVALID;
   if(!aligned16(in) || !aligned16(spec)) return FUFFT_ERR_ALIGN;
   if(!same_or_disjoint({in, (uint64_t)(h * w * batch * 8)}, {spec, (uint64_t)(h * w * batch * 8)}))
      return FUFFT_ERR_INVALID;
   const float2* tw = nullptr;
   if((st = current_table(&tw)) != FUFFT_OK) return st;
   if(batch == 0) return FUFFT_OK;
   const int64_t np = h * w, sub = subbatch_items(np * 8, batch, SUBBATCH_2D_MB);
   for(int64_t i0 = 0; i0 < batch; i0 += sub) {
      const int64_t nb = batch - i0 < sub ? batch - i0 : sub;
      char* dst = static_cast<char*>(spec) + i0 * np * 8;
      Conv1dParams r = rows_params(tw, h, nb);
      r.in0 = static_cast<const char*>(in) + i0 * np * 8; r.out0 = dst;
      if((st = run_conv1d(K_FWD, (int)w, pl.vr, r, stream)) != FUFFT_OK) return st;
      ColParams c = col_params(tw, w, nb);
      c.in = dst; c.out = dst;
      const hipError_t e = launch_col(COL_FWD, (int)h, c, static_cast<hipStream_t>(stream));
      if(e != hipSuccess) return status_of(e);
   }
   return FUFFT_OK;
}

int fufft_apply2d_f32(const void* spec, int64_t spec_stride, const void* filt, int64_t filt_stride,
                      void* out, int64_t h, int64_t w, int64_t batch, int mid, int layout,
                      void* stream)
{
   Plan2d pl;
   int st = check_2d(h, w, batch, &pl);
   if(st != FUFFT_OK) return st;
   if(pl.small) return FUFFT_ERR_UNSUPPORTED;      // the fused conv only, as in the reference
   if(!mid_known(mid) || !layout_ok(layout)) return FUFFT_ERR_INVALID;
   if(!spec || !out || (mid_needs_filter(mid) && !filt)) return FUFFT_ERR_INVALID;
   if(!aligned16(spec) || !aligned16(out) || (filt && !aligned16(filt))) return FUFFT_ERR_ALIGN;
   const int64_t np = h * w;
   if((filt_stride != 0 && filt_stride != np) || (spec_stride != 0 && spec_stride != np))
      return FUFFT_ERR_INVALID;
   // in place only with one spectrum per image: a spectrum shared by the
   // batch would be overwritten by the first image while the others read it
   {
      const Span ss{spec, per_item_bytes(spec_stride, batch, np * 8)}, so{out, (uint64_t)(np * batch * 8)};
      const Span sf{mid_needs_filter(mid) ? filt : nullptr, per_item_bytes(filt_stride, batch, np * 8)};
      if(!same_or_disjoint(ss, so) || !disjoint(so, sf)) return FUFFT_ERR_INVALID;
   }
   const float2* tw = nullptr;
   if((st = current_table(&tw)) != FUFFT_OK) return st;
   if(batch == 0) return FUFFT_OK;
   const int64_t sub = subbatch_items(np * 8, batch, SUBBATCH_2D_MB);
   for(int64_t i0 = 0; i0 < batch; i0 += sub) {
      const int64_t nb = batch - i0 < sub ? batch - i0 : sub;
      char* dst = static_cast<char*>(out) + i0 * np * 8;
      ColParams c = col_params(tw, w, nb);
      set_filter_layout(c, pl, w, layout);
      c.spec = spec_stride == 0 ? spec : static_cast<const char*>(spec) + i0 * np * 8;
      c.out = dst; c.mid = mid;
      c.filt = (filt_stride == 0 || !filt) ? filt : static_cast<const char*>(filt) + i0 * np * 8;
      c.fcount = (uint32_t)(filt_stride == 0 ? 1 : nb);
      c.scount = (uint32_t)(spec_stride == 0 ? 1 : nb);
      const hipError_t e = launch_col(COL_APPLY, (int)h, c, static_cast<hipStream_t>(stream));
      if(e != hipSuccess) return status_of(e);
      Conv1dParams r = rows_params(tw, h, nb);
      r.spec = dst; r.scount = r.ntrans; r.out0 = dst;
      if((st = run_conv1d(K_APPLY, (int)w, pl.vr, r, stream)) != FUFFT_OK) return st;
   }
   return FUFFT_OK;
}

}  // extern "C"
