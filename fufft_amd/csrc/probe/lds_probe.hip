// LDS bank probe for gfx950: every lane of a 64-lane workgroup issues one LDS
// instruction form, REPS times, at the float2 slot the host gives it.  Run
// under rocprofv3 with SQ_LDS_BANK_CONFLICT, one dispatch per (pattern, form),
// it measures the conflict cycles per instruction of that access pattern,
// which is what the LDS layouts of the conv kernels are designed against.
// A diagnostic, not part of the conv library.
#include <hip/hip_runtime.h>

namespace {

constexpr int kSlots = 20480;     // 160 KiB of dynamic LDS, float2 slots

enum { READ_B64 = 0, READ2_B64 = 1, WRITE_B64 = 2, WRITE2_B64 = 3, READ2ST64_B64 = 4 };

template<int FORM>
__global__ void __launch_bounds__(64) lds_probe_kernel(const int* slot, int reps, float* out)
{
   extern __shared__ float2 lds[];
   for(int i = threadIdx.x; i < kSlots; i += 64) lds[i] = make_float2((float)i, 0.f);
   __syncthreads();
   const unsigned a = (unsigned)slot[threadIdx.x] * 8u;
   float acc = 0.f;
   for(int r = 0; r < reps; r++) {
      if constexpr(FORM == READ_B64) {
         float2 v;
         asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
         acc += v.x;
      } else if constexpr(FORM == READ2_B64) {
         float4 v;
         asm volatile("ds_read2_b64 %0, %1 offset1:1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
         acc += v.x + v.z;
      } else if constexpr(FORM == WRITE_B64) {
         const float2 v = make_float2(acc, 1.f);
         asm volatile("ds_write_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : : "v"(a), "v"(v) : "memory");
         acc += 1.f;
      } else if constexpr(FORM == WRITE2_B64) {
         const float2 v = make_float2(acc, 1.f), w = make_float2(1.f, acc);
         asm volatile("ds_write2_b64 %0, %1, %2 offset1:1\n\ts_waitcnt lgkmcnt(0)" : : "v"(a), "v"(v), "v"(w) : "memory");
         acc += 1.f;
      } else {
         float4 v;
         asm volatile("ds_read2st64_b64 %0, %1 offset1:1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
         acc += v.x + v.z;
      }
   }
   out[blockIdx.x * 64 + threadIdx.x] = acc;
}

}  // namespace

// slot: 64 device ints, each < kSlots - 64 (the second access of read2st64 is
// 64 slots further).  out: blocks * 64 floats.  Returns a hipError_t.
extern "C" int fufft_lds_probe(int form, const int* slot, int reps, float* out, int blocks, void* stream)
{
   const void* k = form == READ_B64   ? (const void*)&lds_probe_kernel<READ_B64>
                 : form == READ2_B64  ? (const void*)&lds_probe_kernel<READ2_B64>
                 : form == WRITE_B64  ? (const void*)&lds_probe_kernel<WRITE_B64>
                 : form == WRITE2_B64 ? (const void*)&lds_probe_kernel<WRITE2_B64>
                 : form == READ2ST64_B64 ? (const void*)&lds_probe_kernel<READ2ST64_B64> : nullptr;
   if(!k || !slot || !out || reps < 0 || blocks <= 0) return (int)hipErrorInvalidValue;
   const size_t shm = kSlots * sizeof(float2);
   hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
   if(e != hipSuccess) return (int)e;
   void* args[] = { &slot, &reps, &out };
   return (int)hipLaunchKernel(k, dim3(blocks), dim3(64), args, shm, static_cast<hipStream_t>(stream));
}
