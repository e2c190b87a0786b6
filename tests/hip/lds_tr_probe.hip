// Test-only probe: what ds_read_b64_tr_b16 returns to each lane.
//
// One wave fills a 16 x 64 bf16 LDS matrix with element (r, c) = r*64 + c
// (exact in bf16 up to 256; values are stored as ushort indices instead), then
// every lane issues one transpose read at the address the GEMM kernels use
// for k-block 0 of a 32x32x16 operand, and writes the 4 ushorts it received.
// All addresses stay inside the 2 KiB matrix.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

__global__ void tr_probe_kernel(uint16_t* out) {
  __shared__ __attribute__((aligned(16))) uint16_t m[16 * 64];
  const int lane = threadIdx.x;
  for (int i = lane; i < 16 * 64; i += 64) m[i] = static_cast<uint16_t>(i);
  __syncthreads();
  const int g = lane >> 4, i = lane & 15;
  const int row = (g >> 1) * 8 + (i >> 2);
  const int col = (g & 1) * 16 + (i & 3) * 4;
  const bf16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(m + row * 64 + col));
  reinterpret_cast<uint2*>(out)[lane] = __builtin_bit_cast(uint2, v);
}

extern "C" int ffmoe_probe_lds_tr(void* out_dev) {
  hipLaunchKernelGGL(tr_probe_kernel, dim3(1), dim3(64), 0, 0, static_cast<uint16_t*>(out_dev));
  if (hipGetLastError() != hipSuccess) return 1;
  return hipDeviceSynchronize() == hipSuccess ? 0 : 1;
}
