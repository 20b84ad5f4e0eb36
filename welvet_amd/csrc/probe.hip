// probe.hip — a streaming-read bandwidth probe for bench.py (`--workload
// stream_read`), built as its own library (libwv_probe.so): not part of the
// C ABI. One launch reads `bytes` (a multiple of 4096) with one non-temporal
// 16-byte load per thread, 256 threads per block, one block per 4 KiB: the
// plainest decomposition of one HBM stream into a grid, i.e. the ceiling a
// single launch of that size reaches on this GPU, against which the GEMV's
// fraction of 8 TB/s can be read.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256) k_stream_read(const u32x4* __restrict__ p, uint32_t* __restrict__ sink) {
    const u32x4 v = __builtin_nontemporal_load(p + int64_t(blockIdx.x) * 256 + threadIdx.x);
    // never true for the zero-filled buffers bench.py passes; keeps the load live
    if ((v.x ^ v.y ^ v.z ^ v.w) == 0x9e3779b9u) sink[0] = v.x;
}

}  // namespace

extern "C" int wv_probe_stream_read(const void* buf, size_t bytes, void* sink, void* stream) {
    if (!buf || !sink || bytes == 0 || bytes % 4096) return -1;
    hipLaunchKernelGGL(k_stream_read, dim3(unsigned(bytes / 4096)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const u32x4*>(buf), static_cast<uint32_t*>(sink));
    return hipGetLastError() == hipSuccess ? 0 : -5;
}
