// Quantize-on-append into the fp8 cache-row format (SAS_KV_FP8_DS_MLA).
//
// The reference keeps its caches in bf16/fp16 (api.py:51-56) and has no fp8
// writer; this kernel produces the 656-byte rows the attention kernel reads:
//   bytes [0, 512)   e4m3 of dims 0..511, block t = dims 128t..128t+127
//   bytes [512, 528) fp32 scale of each block: amax / 448 (1 for an all-zero block)
//   bytes [528, 656) dims 512..575 copied as bf16
// e4m3[d] = rne_e4m3(clamp(x[d] / scale, -448, 448)) with an IEEE fp32 division;
// v_cvt_pk_fp8_f32 rounds to nearest even in the OCP e4m3 format (no
// infinities; 448 is the largest finite value).
//
// One wave per row: lane l converts dims 8l..8l+7 (16 lanes per block, so the
// block amax is a 16-lane reduction) and lanes 0..15 copy the rope bytes.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/sas_mi355x.h"

namespace sas {

void set_error(const std::string& msg);

constexpr int FP8_ROWS_PER_WG = 4;
constexpr float E4M3_MAX = 448.0f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(64 * FP8_ROWS_PER_WG) void kv_fp8_append_kernel(
    const __bf16* __restrict__ src, const int32_t* __restrict__ slots,
    unsigned char* __restrict__ cache, int n, int64_t cache_rows) {
  const int row = (int)blockIdx.x * FP8_ROWS_PER_WG + (int)(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n) return;
  const int64_t slot = slots[row];
  if (slot < 0 || slot >= cache_rows) return;
  const __bf16* x = src + (size_t)row * 576;
  const bf16x8 v = *(const bf16x8*)(x + 8 * lane);
  float f[8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    f[i] = (float)v[i];
    amax = fmaxf(amax, fabsf(f[i]));
  }
  // amax over the 16 lanes of this lane's block (xor offsets stay inside the group)
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  const float scale = amax > 0.0f ? amax / E4M3_MAX : 1.0f;
  int packed[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = fminf(fmaxf(f[4 * h + i] / scale, -E4M3_MAX), E4M3_MAX);
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], w, true);
    packed[h] = w;
  }
  unsigned char* out = cache + (size_t)slot * SAS_FP8_ROW_BYTES;
  *(uint2*)(out + 8 * lane) = make_uint2((uint32_t)packed[0], (uint32_t)packed[1]);
  if ((lane & 15) == 0) *(float*)(out + 512 + 4 * (lane >> 4)) = scale;
  if (lane < 16) *(uint2*)(out + 528 + 8 * lane) = *(const uint2*)(x + 512 + 4 * lane);
}

}  // namespace sas

extern "C" int sas_kv_fp8_append(const void* src, const int32_t* slot_mapping, void* cache, int n,
                                 int64_t cache_rows, void* stream) {
  if (n < 0 || cache_rows < 0 || (n > 0 && (!src || !slot_mapping || !cache))) {
    sas::set_error("sas_kv_fp8_append: null pointer or negative size");
    return SAS_E_INVALID;
  }
  if (n == 0) return SAS_OK;
  const int grid = (n + sas::FP8_ROWS_PER_WG - 1) / sas::FP8_ROWS_PER_WG;
  hipLaunchKernelGGL(sas::kv_fp8_append_kernel, dim3(grid), dim3(64 * sas::FP8_ROWS_PER_WG), 0,
                     (hipStream_t)stream, (const __bf16*)src, slot_mapping, (unsigned char*)cache, n,
                     cache_rows);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    sas::set_error(std::string("sas_kv_fp8_append: ") + hipGetErrorString(e));
    return SAS_E_HIP;
  }
  return SAS_OK;
}
