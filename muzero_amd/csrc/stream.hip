// Streaming-read probe (gfx950, wave64): reads a device buffer once and
// XOR-folds it into one word per workgroup.  It moves the bytes a decode or
// quantize kernel would read, with no other work, so its rate is the read
// bandwidth a streaming kernel attains on the device it runs on: the
// measurement that the decode kernels' rates are set against, beside the
// published 8 TB/s peak.  Each workgroup reads one contiguous slab with four
// 16-byte loads per lane in flight.
#include "common.hpp"

namespace mz {

constexpr int SR_WG = 256;
typedef uint32_t sr_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t fold4(const sr_u32x4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

__global__ __launch_bounds__(SR_WG) void stream_read_kernel(const sr_u32x4* __restrict__ p, int64_t n16,
                                                           uint32_t* __restrict__ out) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t beg = per * blockIdx.x;
  const int64_t end = beg + per < n16 ? beg + per : n16;
  uint32_t acc = 0;
  int64_t i = beg + threadIdx.x;
  for (; i + 3 * SR_WG < end; i += 4 * SR_WG) {
    const sr_u32x4 v0 = __builtin_nontemporal_load(p + i);
    const sr_u32x4 v1 = __builtin_nontemporal_load(p + i + SR_WG);
    const sr_u32x4 v2 = __builtin_nontemporal_load(p + i + 2 * SR_WG);
    const sr_u32x4 v3 = __builtin_nontemporal_load(p + i + 3 * SR_WG);
    acc ^= fold4(v0) ^ fold4(v1) ^ fold4(v2) ^ fold4(v3);
  }
  for (; i < end; i += SR_WG) acc ^= fold4(__builtin_nontemporal_load(p + i));
  // workgroup fold: the wave's lanes, then the waves through LDS
  for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, 64);
  __shared__ uint32_t part[SR_WG / 64];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
    for (int w = 0; w < SR_WG / 64; ++w) t ^= part[w];
    out[blockIdx.x] = t;
  }
}

}  // namespace mz

extern "C" int muzero_stream_read(const void* src, int64_t bytes, uint32_t* out, int n_out, mz_stream_t stream) {
  if ((!src && bytes) || !out || bytes < 0 || bytes % 16 != 0 || (uintptr_t)src % 16 != 0 || n_out < 1 || n_out > 65535)
    return MZ_EINVAL;
  mz::stream_read_kernel<<<n_out, mz::SR_WG, 0, (hipStream_t)stream>>>((const mz::sr_u32x4*)src, bytes / 16, out);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MZ_OK : (int)e;
}
