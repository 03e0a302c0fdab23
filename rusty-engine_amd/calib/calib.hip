// Machine calibration kernels for bench.py (not part of the product ABI): streaming reads of a
// device buffer (interleaved over the grid, or one contiguous run per workgroup), a
// dependency-free MFMA stream and an empty kernel. bench.py times them with HIP
// events to measure what this GPU reaches (HBM read bandwidth with the default and the
// nontemporal cache policy, bf16 MFMA throughput, the per-launch floor of a graph of kernels).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

// Every thread reads 16-byte words i = tid, tid + stride, ... below n16 (in bounds by the loop
// test) with buffer loads, eight in flight, and folds them with xor; one word per thread is
// written to sink (tid < threads: sink holds gridDim * 256 words) so the loads are kept.
template <int AUX>
__global__ __launch_bounds__(256) void stream_read_kernel(const uint8_t* p, uint64_t bytes, uint32_t* sink) {
  const uint64_t n16 = bytes / 16;
  const uint64_t tid = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  uint32_t acc = 0;
  uint64_t i = tid;
  for (; i + 7 * stride < n16; i += 8 * stride) {
    i32x4_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint64_t o = (i + (uint64_t)j * stride) * 16;
      // the resource's base moves in 1 GiB windows so the 32-bit offset stays in range
      const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t*>(p) + (o & ~((uint64_t)(1u << 30) - 1)), (short)0, (int)0x7fffffff, 0x00020000);
      v[j] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(o & ((1u << 30) - 1)), 0, AUX);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= (uint32_t)(v[j][0] ^ v[j][1] ^ v[j][2] ^ v[j][3]);
  }
  for (; i < n16; i += stride) {
    const uint64_t o = i * 16;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(p) + (o & ~((uint64_t)(1u << 30) - 1)), (short)0, (int)0x7fffffff, 0x00020000);
    const i32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(o & ((1u << 30) - 1)), 0, AUX);
    acc ^= (uint32_t)(v[0] ^ v[1] ^ v[2] ^ v[3]);
  }
  sink[tid] = acc;
}

// Every workgroup reads its own contiguous run of 16-byte words (bytes / 16 / gridDim words,
// the tail below one run unread), sixteen loads in flight per lane; one word per thread is
// written to sink.
template <int AUX>
__global__ __launch_bounds__(256) void stream_read_chunk_kernel(const uint8_t* p, uint64_t bytes, uint32_t* sink) {
  const uint64_t run = bytes / 16 / gridDim.x;
  const uint64_t b = (uint64_t)blockIdx.x * run;
  uint32_t acc = 0;
  for (uint64_t i = threadIdx.x; i + 15 * 256 < run; i += 16 * 256) {
    i32x4_t v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint64_t o = (b + i + (uint64_t)j * 256) * 16;
      const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t*>(p) + (o & ~((uint64_t)(1u << 30) - 1)), (short)0, (int)0x7fffffff, 0x00020000);
      v[j] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(o & ((1u << 30) - 1)), 0, AUX);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) acc ^= (uint32_t)(v[j][0] ^ v[j][1] ^ v[j][2] ^ v[j][3]);
  }
  sink[(uint64_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

// Each wave runs `iters` rounds of 8 independent v_mfma_f32_32x32x16_bf16 on register operands
// (8 accumulators, no dependency inside a round) and writes one value per wave.
__global__ __launch_bounds__(256) void mfma_stream_kernel(float* out, int iters) {
  const int lane = threadIdx.x & 63;
  bf16x8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(0.001f * (float)(lane + i));
    b[i] = (__bf16)(0.002f * (float)(lane - i));
  }
  f32x16_t acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  if (lane == 0) out[blockIdx.x * 4 + (threadIdx.x >> 6)] = s;
}

__global__ void empty_kernel() {}

}  // namespace

extern "C" {

// bytes of p (a device allocation) read once; sink: grid * 256 words
int cal_stream_read(const void* p, uint64_t bytes, int nontemporal, uint32_t* sink, int grid, void* stream) {
  if (nontemporal)
    hipLaunchKernelGGL(stream_read_kernel<2>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)p, bytes, sink);
  else
    hipLaunchKernelGGL(stream_read_kernel<0>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)p, bytes, sink);
  return (int)hipGetLastError();
}

// the same bytes read as one contiguous run per workgroup (bytes / 16 / grid words each; the
// bytes read are grid * that * 16)
int cal_stream_read_chunk(const void* p, uint64_t bytes, int nontemporal, uint32_t* sink, int grid, void* stream) {
  if (nontemporal)
    hipLaunchKernelGGL(stream_read_chunk_kernel<2>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)p, bytes, sink);
  else
    hipLaunchKernelGGL(stream_read_chunk_kernel<0>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)p, bytes, sink);
  return (int)hipGetLastError();
}

// grid workgroups of 4 waves; out: grid * 4 floats; FLOP = grid * 4 * iters * 8 * 32768
int cal_mfma(float* out, int grid, int iters, void* stream) {
  hipLaunchKernelGGL(mfma_stream_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, out, iters);
  return (int)hipGetLastError();
}

int cal_empty(void* stream) {
  hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream);
  return (int)hipGetLastError();
}

}  // extern "C"
