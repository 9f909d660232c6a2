// Measurement kernels of bench.py (built into libnf4_probe.so, not the NF4 library): what this
// device sustains, for fractions of measured peaks beside the data-sheet ones (the MFMA rate on
// register operands, the HBM read rate).  No counterpart in the reference.
//
//   nf4_probe_mfma(operands, workgroups, iters, dtype, out, stream): `workgroups` x 256 threads
//     issue `iters` x 4 back-to-back v_mfma_f32_32x32x16 (dtype 0 f16, 1 bf16) per wave on
//     operands read from `operands` (>= 128 16-byte vectors), one float per thread to out:
//     2 * 32 * 32 * 16 * 4 * iters * 4 * workgroups flops per launch.
//   nf4_probe_read(src, bytes, workgroups, out, stream): reads `bytes` (a multiple of 16) with
//     16-byte loads over `workgroups` x 256 threads, one uint32 per thread to out.
// Both return 0, or nonzero for bad arguments or a launch error.

#include "../csrc/nf4_common.h"

namespace {

// Back-to-back v_mfma_f32_32x32x16 on four independent accumulators per wave (the matrix
// unit's latency is covered), operands from a buffer (their bit patterns set the power draw),
// one float per thread written so that nothing is optimized away.
template <int DT>
__global__ __launch_bounds__(256) void probe_mfma_kernel(const u32x4_t *operands, int64_t iters,
                                                         float *out) {
    const int lane = threadIdx.x & 63;
    const u32x4_t a = operands[lane], b = operands[64 + lane];
    float16_t acc[4] = {};
    for (int64_t i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (DT == NF4_BF16)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf168_t, a),
                                                                 __builtin_bit_cast(bf168_t, b),
                                                                 acc[j], 0, 0, 0);
            else
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a),
                                                                __builtin_bit_cast(half8_t, b),
                                                                acc[j], 0, 0, 0);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += acc[j][e];
    out[static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x] = s;
}

// Streaming read: 16-byte loads, four in flight per thread, grid-strided; each thread writes
// the XOR of what it read.
__global__ __launch_bounds__(256) void probe_read_kernel(const u32x4_t *src, int64_t n16,
                                                         uint32_t *out) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    uint32_t x = 0;
    int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4_t v0 = src[i], v1 = src[i + stride], v2 = src[i + 2 * stride],
                      v3 = src[i + 3 * stride];
        x ^= v0.x ^ v0.y ^ v0.z ^ v0.w ^ v1.x ^ v1.y ^ v1.z ^ v1.w;
        x ^= v2.x ^ v2.y ^ v2.z ^ v2.w ^ v3.x ^ v3.y ^ v3.z ^ v3.w;
    }
    for (; i < n16; i += stride) {
        const u32x4_t v = src[i];
        x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    out[static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x] = x;
}

}  // namespace

extern "C" int nf4_probe_mfma(const void *operands, int workgroups, int64_t iters, int dtype,
                              float *out, void *stream) {
    if ((dtype != NF4_F16 && dtype != NF4_BF16) || workgroups < 1 || iters < 0 || !operands ||
        !out || !aligned(operands, 16))
        return NF4_ERR_ARG;
    auto s = static_cast<hipStream_t>(stream);
    auto ops = static_cast<const u32x4_t *>(operands);
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL(probe_mfma_kernel<NF4_BF16>, dim3(workgroups), dim3(256), 0, s, ops,
                           iters, out);
    else
        hipLaunchKernelGGL(probe_mfma_kernel<NF4_F16>, dim3(workgroups), dim3(256), 0, s, ops,
                           iters, out);
    return status_of(hipGetLastError());
}

extern "C" int nf4_probe_read(const void *src, int64_t bytes, int workgroups, uint32_t *out,
                              void *stream) {
    if (!src || !out || bytes < 0 || bytes % 16 != 0 || workgroups < 1 || !aligned(src, 16))
        return NF4_ERR_ARG;
    auto s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(probe_read_kernel, dim3(workgroups), dim3(256), 0, s,
                       static_cast<const u32x4_t *>(src), bytes / 16, out);
    return status_of(hipGetLastError());
}
