// Probe of v_mfma_scale_f32_16x16x128_f8f6f4 (e4m3 x e4m3, unit scales) on MI355X:
// one wave per case; A [16 rows][128] and B [16 columns][128] e4m3 codes in (lane
// group g of the wave holds bytes 32 g .. 32 g + 31 of its row / column, the
// layout the attention kernel's fp8 Q·Kᵀ form uses), D [16][16] fp32 out with
// D[r][c] = the MFMA's dot product of A row r and B column c.
// Input file: int32 case count n, then n x 2048 bytes of A, then n x 2048 of B.
// Output file: n x 256 fp32. Built and run by make_fp8_mfma_probe.py.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <cstdint>
#include <vector>
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
__global__ void probe(const uint8_t* A, const uint8_t* B, float* D, int ncase) {
  const int c = blockIdx.x;
  if (c >= ncase) return;
  const int l = threadIdx.x;
  const int r = l & 15, g = l >> 4;
  const uint8_t* a = A + (size_t)c * 2048 + r * 128 + 32 * g;
  const uint8_t* b = B + (size_t)c * 2048 + r * 128 + 32 * g;
  i32x8 x, y;
  for (int i = 0; i < 8; ++i) {
    x[i] = *(const int*)(a + 4 * i);
    y[i] = *(const int*)(b + 4 * i);
  }
  f32x4 d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(x, y, (f32x4){0.f, 0.f, 0.f, 0.f},
                                                             0, 0, 0, 0, 0, 0);
  // lane l: column l % 16, rows 4 g + i
  for (int i = 0; i < 4; ++i) D[(size_t)c * 256 + (4 * g + i) * 16 + r] = d[i];
}
int main(int argc, char** argv) {
  const char* in = argv[1];
  const char* out = argv[2];
  FILE* f = fopen(in, "rb");
  if (!f) { printf("cannot open %s\n", in); return 1; }
  int ncase = 0;
  fread(&ncase, 4, 1, f);
  std::vector<uint8_t> A((size_t)ncase * 2048), B((size_t)ncase * 2048);
  fread(A.data(), 1, A.size(), f);
  fread(B.data(), 1, B.size(), f);
  fclose(f);
  uint8_t *dA, *dB;
  float* dD;
  hipMalloc(&dA, A.size());
  hipMalloc(&dB, B.size());
  hipMalloc(&dD, (size_t)ncase * 256 * 4);
  hipMemcpy(dA, A.data(), A.size(), hipMemcpyHostToDevice);
  hipMemcpy(dB, B.data(), B.size(), hipMemcpyHostToDevice);
  hipLaunchKernelGGL(probe, dim3(ncase), dim3(64), 0, 0, dA, dB, dD, ncase);
  std::vector<float> D((size_t)ncase * 256);
  hipError_t e = hipMemcpy(D.data(), dD, D.size() * 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess) { printf("hip error %s\n", hipGetErrorString(e)); return 1; }
  f = fopen(out, "wb");
  fwrite(D.data(), 4, D.size(), f);
  fclose(f);
  printf("ok %d cases\n", ncase);
  return 0;
}
