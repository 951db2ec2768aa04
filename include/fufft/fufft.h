/*
 * fuFFT for MI355X (gfx950) -- C ABI of the fused cyclic-convolution path.
 *
 * The reference (weiwang217/FuFFT) has no library: its interface is a set of
 * CUDA kernel templates launched by its benchmark driver, plus the host-side
 * planning that driver does.  Each entry point below replaces one of those
 * launches (or one piece of that planning) and cites it.  Conventions:
 *
 *   - Device pointers are caller-owned; nothing here allocates device memory
 *     on the hot path.  The first call on a device uploads the twiddle table
 *     (a one-time synchronous copy into static device memory); call
 *     fufft_init() up front to keep that out of timed or captured regions.
 *   - Complex data is interleaved fp32 (re, im), 8 bytes per point, 16-byte
 *     aligned base pointers.
 *   - stream is a hipStream_t (NULL = the default stream).  Calls are
 *     asynchronous, stateless and thread-safe across streams.
 *   - Every function returns FUFFT_OK (0) or a negative status; none exits.
 *     HIP launch errors are reported as FUFFT_ERR_HIP.
 *   - The device buffers of one call either coincide, where the call says
 *     it works in place (in == out and the like), or share no byte.  Any
 *     other overlap (an output reaching into an input, the filter or another
 *     output) returns FUFFT_ERR_INVALID before anything is launched.
 *   - Filters are spectra with 1/N already folded in, in the digit order the
 *     forward DIF leaves behind (see fufft_plan_filter_f32).  filt_stride is 0
 *     (one filter shared by the batch) or n (one filter per signal).
 *
 * Supported sizes (fufft_supported): single-launch N = 2^k with
 * 256 <= N <= 16384 for FUFFT_V16 and 512 <= N <= 8192 for FUFFT_R8, and the
 * fused conv (fufft_conv_f32) also at N = 32768 for FUFFT_V16; the four-step
 * path takes N = 16^L * MID up to 2^20.
 */
#ifndef FUFFT_FUFFT_H
#define FUFFT_FUFFT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- ABI version ----------------------------------------------------------
 * Bumped whenever an entry point's arguments or the meaning of an id change,
 * so that a caller built against one header can refuse a library built from
 * another (compare fufft_abi_version() with FUFFT_ABI_VERSION):
 *   2  FUFFT_LAYOUT_LANE (1) became the lane-major pair layout (the one-value
 *      lane-major layout moved to FUFFT_LAYOUT_BPERM, 2); the 2D calls and
 *      fufft_conv_r2_f32 gained `layout`;
 *   3  the four-step calls (fufft_large_digit_order, fufft_plan_filter_large_
 *      f32 and _device_f32, fufft_conv_large_f32) gained `variant`, and the
 *      default four-step middle is the reference's radix-16 one;
 *   4  fufft_stream_shape_f32 gained `lanes` (workgroup size).
 * No reference counterpart (the reference ships no library). */
#define FUFFT_ABI_VERSION 4
int fufft_abi_version(void);

/* ---- status -------------------------------------------------------------- */
#define FUFFT_OK                0
#define FUFFT_ERR_INVALID      -1   /* null pointer, bad count, stride or enum */
#define FUFFT_ERR_UNSUPPORTED  -2   /* size / variant combination not built    */
#define FUFFT_ERR_HIP          -3   /* HIP runtime error (init, launch)        */
#define FUFFT_ERR_ALIGN        -4   /* misaligned pointer (16 B fp32, 4 B BFP)  */
#define FUFFT_ERR_SCRATCH      -5   /* one image larger than the static scratch
                                       (fufft_conv2d_r2_noalloc_f32)            */

/* ---- enums ----------------------------------------------------------------- */
/* mid operation between forward and inverse (Mid policies, fufft.cuh:616-650).
 * Each id names a policy struct registered in the library's kernel sources
 * (FUFFT_MID_POLICIES in fufft_amd/csrc/fufft_plan.hpp): as in the reference,
 * a new fusion costs a struct, plus its id here; every call that takes `mid`
 * then accepts it.  fufft_mid_reads_filter tells a caller of a given build
 * which ids exist and which read a filter. */
#define FUFFT_MID_MUL   0   /* A * B        convolution  (MidMultiply)      */
#define FUFFT_MID_CONJ  1   /* A * conj(B)  correlation  (MidConjMultiply)  */
#define FUFFT_MID_NONE  2   /* round trip, N * input      (MidNothing)       */

/* lane layout / radix family */
#define FUFFT_V16  0   /* 16 values per lane, radix 16 (fufft_pipeline_v16)  */
#define FUFFT_R8   1   /* 8 values per lane, radix 8 (fufft_pipeline_ip)     */
#define FUFFT_AUTO 2   /* the faster of the two for this N on MI355X with
                          the digit-order filter (FUFFT_LAYOUT_DR), one rule
                          for the fp32 and the BFP conv: FUFFT_R8 at N = 512,
                          4096 and 8192, FUFFT_V16 elsewhere.  The filter must
                          be planned with the same variant.  For the
                          lane-major filter see fufft_fastest_variant. */

/* filter layouts */
#define FUFFT_LAYOUT_DR    0  /* slot i holds bin mixedrev(i) (MidMultiply, fufft.cuh:635) */
#define FUFFT_LAYOUT_LANE  1  /* lane-major pairs, T = N/V: the values of slots
                                 V*L+2m and V*L+2m+1 at 2(L+m*T) and 2(L+m*T)+1,
                                 so every 16-byte filter load of a wavefront
                                 reads one contiguous KiB (the bperm layout of
                                 fufft_pipeline_v16f, fufft.cuh:1444-1446, is
                                 lane-major one value at a time).  With it
                                 FUFFT_V16 is the fastest variant at
                                 N = 1024 .. 8192 and FUFFT_R8 at N = 512. */
#define FUFFT_LAYOUT_BPERM 2  /* the reference's bperm (fufft_pipeline_v16f,
                                 fufft.cuh:1444-1446; verify_kernel.cpp:
                                 1381-1387): the value of slot V*L+k at
                                 L+k*(N/V).  1D calls only; a filter built for
                                 the reference's _v16f passes as it is. */

/* filter_kind for fufft_plan_filter_f32 */
#define FUFFT_FILTER_SPECTRUM  0  /* input is a natural-order spectrum             */
#define FUFFT_FILTER_TAPS      1  /* input is time-domain taps; DFT taken in fp64  */

/* ---- library ---------------------------------------------------------------- */
/* Upload the twiddle table to `device` (idempotent, thread-safe). */
int fufft_init(int device);
const char* fufft_status_string(int status);
/* 1 if a single-launch kernel exists for (n, variant), else 0.  At
 * n = 32768 (FUFFT_V16) that is the fused conv, fufft_conv_f32, alone; the
 * other 1D calls return FUFFT_ERR_UNSUPPORTED there. */
int fufft_supported(int64_t n, int variant);
/* The faster variant (FUFFT_R8 or FUFFT_V16) for an n-point conv whose filter
 * is in `layout`, as measured on MI355X for the fp32 and the BFP conv alike;
 * FUFFT_AUTO is this for FUFFT_LAYOUT_DR.  With FUFFT_LAYOUT_LANE it is
 * FUFFT_R8 at n = 512 and FUFFT_V16 at every other n, the fastest plan of
 * this library at n = 1024 .. 32768.  Plan the filter and launch with the
 * variant it returns.  No reference counterpart (the reference's caller
 * picks the kernel template). */
int fufft_fastest_variant(int64_t n, int layout);
/* 1 if `mid` is a mid policy of this build that reads a filter (the filter
 * pointer must then be valid), 0 if it is one that reads none (the filter
 * pointer may be NULL), FUFFT_ERR_INVALID if no policy has that id.  No
 * reference counterpart (there a policy is a type the caller instantiates). */
int fufft_mid_reads_filter(int mid);

/* ---- host planning (no GPU needed) ------------------------------------------
 * Pass plan in DIF order: lead radix first, then radix 16 (or 8); returns the
 * pass count or a negative status.  (cpu_mixed.cpp:36-49, bench_fufft.cu:129-134) */
int fufft_plan_radices(int64_t n, int variant, int* radices /* >= 32 */);
/* perm[i] = spectrum bin held by slot i after the forward DIF: bit-group
 * reversal over the radix widths in pass order.
 * (mixedrev_host, bench_fufft.cu:63-82; chain_rev, verify_kernel.cpp:460-477) */
int fufft_digit_order(int64_t n, int variant, int32_t* perm);

/* How each pass of the plan (in plan_radices order) generates its stage
 * twiddles from the base twiddle W^j: FUFFT_CHAIN_SINGLE (W^(jk) =
 * W^(j(k-1)) W^j, fufft.cuh:436-450) or FUFFT_CHAIN_EVENODD (radix 16: even
 * and odd chains, fufft.cuh:701-720).  Returns the pass count. */
#define FUFFT_CHAIN_SINGLE  0
#define FUFFT_CHAIN_EVENODD 1
int fufft_plan_chains(int64_t n, int variant, int* chains /* >= 32 */);
/* Turn a natural-order spectrum or time-domain taps (n complex) into the
 * filter a conv call reads: fp64 DFT for taps, optional 1/n fold, digit-order
 * permutation, optional lane-major layout.  Host memory in and out.
 * (bench_fufft.cu:156-170, verify_kernel.cpp:1381-1387) */
int fufft_plan_filter_f32(int64_t n, int variant, int layout, int filter_kind,
                          int fold_inv_n, const float* in, float* out);
/* The device twiddle table, recomputed on the host: for every P = 2^p,
 * 1 <= p <= log_max, entries [P, 2P) hold (cos, sin)(2*pi*t/P) rounded to
 * fp32.  out must hold 2 * 2^(log_max+1) floats. */
int fufft_twiddle_table_host(int log_max, float* out);

/* Source of the base twiddles W^j every kernel reads from the device table.
 *   FUFFT_TWIDDLES_ACCURATE   (default) (cos, sin)(2*pi*t/P) evaluated in
 *                             fp64 and rounded to fp32.
 *   FUFFT_TWIDDLES_REFERENCE  cosf / sinf of the fp32 angle (2*pi/P)*t, the
 *                             value the reference's device code computes with
 *                             __sincosf(step*j) and its CPU transcription with
 *                             cosf/sinf (fufft.cuh:362-371, 731;
 *                             verify_kernel.cpp:31, 93-99).  With it the fp32
 *                             kernels reproduce that transcription
 *                             (kernel_pipeline_v16 / _ip / _fwd / _apply,
 *                             kernel_conv2d, kernel_conv_r2, the four-step
 *                             chain) bit for bit on the same inputs.
 * fufft_set_twiddles rewrites the table of `device` (a synchronous copy after
 * a device-wide synchronisation): call it while no fufft work is queued on
 * the device and outside stream capture.  The setting holds for every later
 * call on that device. */
#define FUFFT_TWIDDLES_ACCURATE   0
#define FUFFT_TWIDDLES_REFERENCE  1
int fufft_set_twiddles(int device, int source);
int fufft_get_twiddles(int device, int* source);
/* fufft_twiddle_table_host for either source */
int fufft_twiddle_table_host_source(int log_max, int source, float* out);

/* ---- fp32 fused convolution ------------------------------------------------
 * out = IDFT(DFT(in) mid filt) for batch signals of n points, one launch,
 * three HBM passes.  in == out is allowed.  At n = 32768 (FUFFT_V16 or
 * FUFFT_AUTO) one workgroup holds a transform, 32 values per lane, with the
 * radix-16 plan's arithmetic and filter: the filter is the one
 * fufft_plan_filter_f32 writes for (32768, FUFFT_V16) in any of the three
 * layouts, and the result equals that plan bit for bit.  (The four-step call,
 * fufft_conv_large_f32, is the reference's run_large chain at that size.)
 * Replaces fufft_pipeline_v16<N,LEAD,NRV,CPB> (fufft.cuh:1518-1534),
 * fufft_pipeline_v16f (fufft.cuh:1499-1516) and
 * fufft_pipeline_ip<N,LEAD,NR8,CPB,Mid> (fufft.cuh:1757-1772), launched by
 * run_conv (bench_fufft.cu:215-221). */
int fufft_conv_f32(const void* in, const void* filt, int64_t filt_stride,
                   void* out, int64_t n, int64_t batch, int mid, int variant,
                   int layout, void* stream);

/* ---- in-kernel phase timer -----------------------------------------------------
 * fufft_conv_f32 with a timestamp after each phase, for per-phase evidence of
 * where a fused launch spends its time.  The reference's FUFFT_TIMER_* marks
 * (fufft.cuh:86-176, K_LOAD / K_FWD / K_MULT / K_INV / K_STORE, %smid) as a
 * separate entry point instead of a compile-time switch.  Each mark waits for
 * the workgroup's outstanding memory operations and a workgroup barrier, then
 * reads the shader clock (s_memtime), so the timed launch is slower than the
 * untimed one; read proportions and confirm totals against fufft_conv_f32.
 * The output is bit-identical to fufft_conv_f32.
 * Workgroup g (transforms [g*tpw, (g+1)*tpw), tpw from
 * fufft_transforms_per_workgroup) writes, for g < timing_groups, the
 * FUFFT_TIMER_STRIDE words at timing + g*FUFFT_TIMER_STRIDE (device memory):
 *   [0] HW_ID register of the wavefront that wrote the record (gfx9 layout:
 *       wave [3:0], SIMD [5:4], CU [11:8], shader array and engine above),
 *   [1] XCC_ID register (XCD [3:0]), [2] number of marks (5),
 *   [3] ticks of the constant 100 MHz clock (s_memrealtime) from the start
 *       to the last mark, so [10]'s cycles / ([3] / 100 MHz) is the shader
 *       clock the workgroup ran at,
 *   [4], [5] start time (s_memtime), low and high word,
 *   [6 .. 10] phase << 24 | cycles since start (saturated at 2^24 - 1) for
 *   phases 1 load, 2 forward DIF, 3 mid operation, 4 inverse DIT, 5 store.
 * Default LDS layouts only (not FUFFT_LDS_LAYOUT=xor); a call that would need
 * more than one launch (per-signal filters beyond 4 GiB) returns
 * FUFFT_ERR_UNSUPPORTED. */
#define FUFFT_TIMER_STRIDE 12
int fufft_transforms_per_workgroup(int64_t n, int variant);
int fufft_conv_timed_f32(const void* in, const void* filt, int64_t filt_stride,
                         void* out, int64_t n, int64_t batch, int mid, int variant,
                         int layout, uint32_t* timing, int64_t timing_groups,
                         void* stream);

/* ---- split path: one signal against many filters ----------------------------
 * fwd: natural-order signal -> digit-order spectrum (fufft_pipeline_fwd,
 * fufft.cuh:1343-1370).  apply: spectrum (spec_stride 0 = one spectrum for
 * the whole batch, n = one per item) mid filt -> inverse -> natural order
 * (fufft_pipeline_apply, fufft.cuh:1372-1407).  fwd followed by apply is
 * bit-identical to fufft_conv_f32. */
int fufft_fwd_f32(const void* in, void* spec, int64_t n, int64_t batch,
                  int variant, void* stream);
int fufft_apply_f32(const void* spec, int64_t spec_stride, const void* filt,
                    int64_t filt_stride, void* out, int64_t n, int64_t batch,
                    int mid, int variant, int layout, void* stream);

/* ---- two-for-one real convolution --------------------------------------------
 * u = x (*) h, v = y (*) h for real x, y (fp32, n per signal) and a REAL
 * time-domain filter h whose spectrum is filt: both ride one complex
 * transform (fufft_conv_r2, fufft.cuh:1260-1330). */
int fufft_conv_r2_f32(const float* x, const float* y, const void* filt,
                      int64_t filt_stride, float* u, float* v, int64_t n,
                      int64_t batch, int variant, int layout, void* stream);

/* ---- natural-order batched C2C ------------------------------------------------
 * out = DFT(in) with direction FUFFT_FORWARD (exp(-2 pi i jk/n)) or the
 * unnormalised inverse with FUFFT_INVERSE (exp(+2 pi i jk/n)), natural order
 * in and out, batch transforms of n points, one launch, two HBM passes;
 * in == out is allowed.  Replaces fufft_c2c<N,LOG8N,CPB> (fufft.cuh:879-904),
 * a forward-only radix-8 Stockham transform for N = 8^k launched with one
 * workgroup per CPB transforms.  Here the forward DIF of the conv kernels (or
 * their inverse DIT) runs unchanged and one exchange through LDS moves the
 * spectrum between digit order and natural order, for every size and
 * variant fufft_supported accepts. */
#define FUFFT_FORWARD (-1)
#define FUFFT_INVERSE   1
int fufft_c2c_f32(const void* in, void* out, int64_t n, int64_t batch,
                  int direction, int variant, void* stream);

/* ---- filter planning on the device ----------------------------------------------
 * The host planning step of the reference (filter spectrum, digit-order
 * permutation and 1/N fold: bench_fufft.cu:156-170; chain order,
 * bench_fufft.cu:410-428; 2D order, verify_kernel.cpp:738-748) for `count`
 * filters already in device memory.  Same arguments and output as
 * fufft_plan_filter_f32 / _large_ / 2d_ (n, or h*w, complex points per filter).
 *   FUFFT_FILTER_SPECTRUM: a gather into the conv's digit order (times 1/n
 *     with fold_inv_n); bit-identical to the host planner.  in != out.
 *   FUFFT_FILTER_TAPS: the conv kernels' own forward transform in fp32
 *     (times 1/n, exact since n is a power of two).  The host planner takes
 *     this DFT in fp64 instead, so the two agree to fp32 transform rounding
 *     (rel L2 ~3e-7), not bit for bit.  in == out is allowed.
 * In 1D, spectra are planned for every n the fused conv takes (n = 32768
 * included), taps up to n = 16384 (FUFFT_ERR_UNSUPPORTED beyond). */
int fufft_plan_filter_device_f32(const void* in, void* out, int64_t n, int64_t count,
                                 int variant, int layout, int filter_kind,
                                 int fold_inv_n, void* stream);
int fufft_plan_filter_large_device_f32(const void* in, void* out, int64_t n,
                                       int64_t count, int variant, int filter_kind,
                                       int fold_inv_n, void* stream);
int fufft_plan_filter2d_device_f32(const void* in, void* out, int64_t h, int64_t w,
                                   int64_t count, int layout, int filter_kind,
                                   int fold_inv_n, void* stream);

/* ---- int16 block floating point ----------------------------------------------
 * A point is two int16 (re in the low halfword, im in the high halfword);
 * every block of `block` consecutive points of a signal shares one int8
 * exponent e, value = q * 2^e.  Exponent rule: e = -128 for an all-zero
 * (or subnormal) block, else the smallest e with absmax <= 32767 * 2^e,
 * clamped at -128; q = rint(x * 2^-e), so |q| <= 32767.
 * Replaces fufft_pipeline_v16_bfp (fufft.cuh:1614-1701), whose format is one
 * fp32 scale per transform and an int16 filter; here the filter is fp32, and
 * block = n gives one exponent per transform like the reference's scale.
 * FUFFT_BFP_BLOCK is the smallest block (and the bench's). */
#define FUFFT_BFP_BLOCK 64
int fufft_bfp_exponent(float absmax);
/* host reference codec (bfp_quant_host, bench_fufft.cu:105-117); npts a
 * multiple of block */
int fufft_bfp_quantize(const float* x, int64_t npts, int64_t block, int16_t* q, int8_t* e);
int fufft_bfp_dequantize(const int16_t* q, const int8_t* e, int64_t npts, int64_t block,
                         float* x);
/* Fused conv on BFP data: dequantise on load, the fp32 pipeline of
 * fufft_conv_f32 (bit for bit), quantise on store with the rule above.
 * qin / qout: n*batch points (4 bytes each); ein / eout: n*batch/block
 * exponents; block: a power of two, FUFFT_BFP_BLOCK <= block <= n;
 * filt: fp32 filter planned for the same variant.  Needs n/V >= 64 lanes:
 * FUFFT_R8 512..8192, FUFFT_V16 1024..16384.  qin == qout and ein == eout are
 * allowed.  qin, qout, ein and eout must be 4-byte aligned (FUFFT_ERR_ALIGN). */
int fufft_conv_bfp16(const void* qin, const int8_t* ein, const void* filt,
                     int64_t filt_stride, void* qout, int8_t* eout, int64_t n,
                     int64_t batch, int64_t block, int mid, int variant, int layout,
                     void* stream);

/* ---- int16 BFP in the reference's own format -----------------------------------
 * fufft_pipeline_v16_bfp(aq, a_scale, bq, b_scale, outq, out_scale)
 * (fufft.cuh:1614-1701; its CPU transcription kernel_v16_bfp and bfp_quantize,
 * verify_kernel.cpp:1092-1135): int16 pairs as above with one fp32 scale per
 * transform, value = q * scale; the filter is int16 pairs (the fp32 filter of
 * fufft_plan_filter_f32 for the same variant and layout, quantised by
 * fufft_bfp_scaled_quantize) with one fp32 scale per filter.  layout: the
 * reference's digit order FUFFT_LAYOUT_DR, or the slots of FUFFT_LAYOUT_LANE /
 * FUFFT_LAYOUT_BPERM (same values, same result).  On
 * output, per transform: mx = max(abs-max of the fp32 result, 1e-30),
 * q = rint(clamp(v * (32767 / mx), -32767, 32767)), scale = mx / 32767.
 * filt_stride 0: one filter (qfilt n points, sfilt one scale) for the batch;
 * n: one per transform (n*batch points, batch scales).  The fp32 pipeline in
 * between is fufft_conv_f32's, so with FUFFT_TWIDDLES_REFERENCE and
 * FUFFT_V16 the words and scales equal the reference transcription's.
 * FUFFT_V16 256..16384, FUFFT_R8 512..8192 (the reference: FUFFT_V16).
 * qin == qout and sin == sout are allowed.  qin, qout, sin, sout, sfilt
 * 4-byte aligned, qfilt 16-byte aligned (FUFFT_ERR_ALIGN). */
int fufft_conv_bfp16_scaled(const void* qin, const float* sin, const void* qfilt,
                            const float* sfilt, int64_t filt_stride, void* qout, float* sout,
                            int64_t n, int64_t batch, int mid, int variant, int layout,
                            void* stream);
/* host codec of that format (bfp_quantize, verify_kernel.cpp:1092-1105):
 * count transforms of n points, x interleaved re/im, one scale per transform */
int fufft_bfp_scaled_quantize(const float* x, int64_t n, int64_t count, int16_t* q, float* scale);
int fufft_bfp_scaled_dequantize(const int16_t* q, const float* scale, int64_t n, int64_t count,
                                float* x);

/* ---- HBM stream ceiling (measurement) ------------------------------------------------
 * Copies `bytes` (a multiple of 16; 16-byte aligned pointers; in != out) with
 * the buffer instructions the conv kernels use: each 256-lane workgroup moves
 * 32 KiB, eight 16-byte loads per lane in flight before the stores.
 * nontemporal = 1 adds the streaming (NT) cache policy to both.  No
 * counterpart in the reference, which quotes its device's peak bandwidth
 * (bench_fufft.cu:506): bench.py reports this copy's GB/s as the measured HBM
 * ceiling beside MI355X's 8 TB/s, and this copy of known size scales the
 * rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes. */
int fufft_stream_f32(const void* in, void* out, int64_t bytes, int nontemporal, void* stream);
/* The same copy in a chosen shape, so that the ceiling is the best of a sweep
 * of shapes rather than one configuration (same argument rules as above):
 *   lanes            64, 256 or 1024 lanes per workgroup;
 *   load_bytes       8 or 16 bytes per load and store (16: the stream copy
 *                    above; 8: the float2 width of the conv kernels' I/O);
 *   loads_per_lane   1, 2, 4, 8, 16 or 32 loads per lane in flight before
 *                    the stores (a workgroup tile of lanes x that many, at
 *                    most 256 KiB);
 *   tiles_per_group  1..4096 consecutive tiles per workgroup, in a loop;
 *   groups           0, or a persistent grid of that many workgroups that
 *                    stride over the tiles (tiles_per_group is then ignored);
 *   load_policy,     cache-policy bits of the loads and of the stores, 0..3:
 *   store_policy     SC0 = 1, NT = 2 (streaming), as the gfx950 buffer
 *                    instructions take them.
 * fufft_stream_f32 is (256, 16, 8, 1, 0, p, p) with p = 0 or NT.  No
 * reference counterpart (measurement only). */
int fufft_stream_shape_f32(const void* in, void* out, int64_t bytes, int lanes, int load_bytes,
                           int loads_per_lane, int tiles_per_group, int groups,
                           int load_policy, int store_policy, void* stream);

/* ---- four-step large N -------------------------------------------------------------
 * N = 16^lout * mid with mid a single-launch size: lout radix-16 DIF levels
 * over HBM, the fused conv on contiguous mid-point chunks in place, lout DIT
 * levels (run_large / MidLaunch, bench_fufft.cu:357-492;
 * fufft_outer_pass_r, fufft.cuh:1113-1140).  buf is transformed in place.
 * fufft_large_plan gives lout and mid (the fewest outer levels that leave
 * mid <= 4096: 32768 = 16 x 2048, 65536 = 16 x 4096, 262144 = 16^2 x 1024,
 * as run_large's instantiations, bench_fufft.cu:519-520).
 * `variant` names the middle's plan and so the filter's chain order,
 * [16]^lout followed by the middle's radices:
 *   FUFFT_V16 (and FUFFT_AUTO): the reference's middle, fufft_pipeline_v16 on
 *     the chunks, so a filter permuted as run_large permutes it
 *     (bench_fufft.cu:410-428, [16]^lout ++ [lead] ++ [16]^k) passes as it is;
 *   FUFFT_R8: a radix-8 middle ([16]^lout ++ [lead] ++ [8]^k), the chain of
 *     the reference's radix-8 conv_foursteps_cfg (verify_kernel.cpp:373-394).
 * Plan the filter (fufft_large_digit_order, fufft_plan_filter_large_f32 or
 * its device form) and run the conv with the same variant.
 * The reference makes 4*lout + 3 HBM passes; here the two outer levels of a
 * two-level plan (n >= 2^17) run as one pass through LDS, bit-identical, so
 * every plan reads and writes the data three times. */
int fufft_large_plan(int64_t n, int* lout, int* mid);
int fufft_large_digit_order(int64_t n, int variant, int32_t* perm);
int fufft_plan_filter_large_f32(int64_t n, int variant, int filter_kind, int fold_inv_n,
                                const float* in, float* out);
int fufft_conv_large_f32(void* buf, const void* filt, int64_t filt_stride,
                         int64_t n, int64_t batch, int mid, int variant, void* stream);

/* ---- 2D ---------------------------------------------------------------------------
 * h x w images, row-major.  Rows DIF, columns DIF, mid, columns DIT, rows DIT
 * (fufft_conv2d, fufft.cuh:1209-1258).  Two shape ranges:
 *   small images, h * w <= 8192 with h and w powers of two from 8 to 512 (the
 *     reference's own fufft_conv2d shapes are powers of 8 up to 4096 points):
 *     one fused launch per batch, the whole image in one workgroup's LDS,
 *     radix 8 both ways; fufft_conv2d_f32 and the host planner only (the
 *     reference has no split or two-for-one path for them; those calls return
 *     FUFFT_ERR_UNSUPPORTED, as does device planning of taps);
 *   large images, h in 256 .. 2048, w a single-launch 1D size (256 .. 16384):
 *     three launches in place on out: row forward, fused column conv, row
 *     inverse (an image too large for one workgroup).
 * 2D filters: `layout` names the column order of the filter a call reads or
 * a planner writes.
 *   FUFFT_LAYOUT_DR    the reference's order (verify_kernel.cpp:738-748):
 *                      entry (r, c) holds spectrum bin (mixedrev_h(r),
 *                      mixedrev_w(c)).
 *   FUFFT_LAYOUT_LANE  this library's order: entry (r, c) holds bin
 *                      (mixedrev_h(r), mixedrev_w(slot(c))), where slot(c) is
 *                      the row plan's digit-order slot that column c of the
 *                      row spectra holds (fufft_plan2d_column_order): the rows
 *                      are in the 1D FUFFT_LAYOUT_LANE order, column
 *                      c = 2(L + m*T) + j holding slot V*L + 2m + j with V the
 *                      row plan's values per lane and T = w / V, so the row
 *                      kernels store and load whole contiguous runs.  A
 *                      column tile then reads its filter columns as one
 *                      contiguous run per row, which DR order does not give.
 * Both layouts give bit-identical results.  2D spectra (fufft_fwd2d_f32,
 * fufft_apply2d_f32) are always in the FUFFT_LAYOUT_LANE order.  For small
 * images the column order is the identity: both layouts are the reference's. */
/* Values per lane of the row plan (the 1D kernel at FUFFT_AUTO for length w)
 * and of the column plan (8 up to h = 512, 16 for h = 1024, 2048; 8 and 8 for
 * small images); the
 * per-dimension digit orders are those of fufft_digit_order with that many
 * values per lane.  No reference counterpart (the reference fixes both
 * dimensions at compile time, fufft.cuh:1209-1214). */
int fufft_plan2d(int64_t h, int64_t w, int* v_rows, int* v_cols);
/* slot[c] (w entries) = the row plan's digit-order slot held by column c of
 * 2D filters and spectra.  No reference counterpart (a layout of this build). */
int fufft_plan2d_column_order(int64_t h, int64_t w, int32_t* slot);
int fufft_plan_filter2d_f32(int64_t h, int64_t w, int layout, int filter_kind,
                            int fold_inv_n, const float* in, float* out);
int fufft_conv2d_f32(const void* in, const void* filt, int64_t filt_stride,
                     void* out, int64_t h, int64_t w, int64_t batch, int mid,
                     int layout, void* stream);
/* Two real images per complex transform with a REAL filter; work is a
 * caller-owned complex scratch of h*w*batch points (the packed images). */
int fufft_conv2d_r2_f32(const float* x, const float* y, const void* filt,
                        int64_t filt_stride, float* u, float* v, void* work,
                        int64_t h, int64_t w, int64_t batch, int layout,
                        void* stream);
/* Two-for-one 2D conv without a workspace.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results (bit for bit) as fufft_conv2d_r2_f32 without `work`:
 * the packed images go through a static device array of FUFFT_SCRATCH_BYTES
 * that the library holds on every GPU it runs on until the process ends, in
 * sub-batches of at most FUFFT_SCRATCH_BYTES / (8*h*w) images.  An image
 * larger than the array (8*h*w > FUFFT_SCRATCH_BYTES, e.g. 2048 x 8192)
 * returns FUFFT_ERR_SCRATCH.  The call allocates nothing.  Every call on one
 * GPU uses that GPU's one array, which keeps the last call's contents (each
 * call writes every element it reads): calls that overlap on one GPU (two
 * streams, two host threads) race on it and must be serialised.  Call
 * fufft_init(device) first to keep the one-time twiddle upload out of the
 * call and out of graph capture. */
#define FUFFT_SCRATCH_BYTES (64ll << 20)
int fufft_conv2d_r2_noalloc_f32(const float* x, const float* y, const void* filt,
                                int64_t filt_stride, float* u, float* v, int64_t h,
                                int64_t w, int64_t batch, int layout, void* stream);
/* split 2D path: fwd = rows DIF then columns DIF into spec (the 2D order above);
 * apply = spec mid filt, columns DIT, rows DIT into out.  spec_stride 0 shares
 * one spectrum across the batch. */
int fufft_fwd2d_f32(const void* in, void* spec, int64_t h, int64_t w,
                    int64_t batch, void* stream);
int fufft_apply2d_f32(const void* spec, int64_t spec_stride, const void* filt,
                      int64_t filt_stride, void* out, int64_t h, int64_t w,
                      int64_t batch, int mid, int layout, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* FUFFT_FUFFT_H */
