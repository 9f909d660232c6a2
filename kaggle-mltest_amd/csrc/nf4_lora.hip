// LoRA side GEMMs (rank <= 64), the SwiGLU step and the bias gradient for gfx950.
//
// Reference: the LoRA mm's of FusedDecoderLayer (/root/reference/solution/layer.py:875-878,
// 1072-1081), the SwiGLU kernels of the organizers' example reused by RecomputedMLP
// (swiglu.py:15-37; mlp.py:26-39) and the bias gradient of NF4Linear (nf4.py:100-101).
// All accumulate in fp32.  These are small next to the projection GEMMs (about 0.3 % of the
// flops of a Qwen2.5-1.5B layer) and are bound by reading their [M, K] / [M, N] operand once.

#include "nf4_common.h"

namespace {

template <int DT>
__device__ __forceinline__ float ld1(const uint16_t *p) {
    if constexpr (DT == NF4_BF16) return __uint_as_float(static_cast<uint32_t>(*p) << 16);
    else return static_cast<float>(__builtin_bit_cast(half_t, *p));
}

template <int DT>
__device__ __forceinline__ uint16_t st1(float v) {
    if constexpr (DT == NF4_BF16) return __builtin_bit_cast(uint16_t, static_cast<bf16_t>(v));
    else return __builtin_bit_cast(uint16_t, static_cast<half_t>(v));
}

template <int DT>
__device__ __forceinline__ void unpack8(const u32x4_t &v, float (&f)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint16_t lo = w[i] & 0xffff, hi = w[i] >> 16;
        f[2 * i] = ld1<DT>(&lo);
        f[2 * i + 1] = ld1<DT>(&hi);
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

constexpr int kMaxRank = 64;

// t[m][j] = sum_k xd[m][k] * A[j][k].  One wave per row m; lanes stride k by 8 elements.
// Also serves da[m][j] = scale * sum_n dY[m][n] * B[n][j] with `a_rowmajor_rank` = true
// (B is [N, rank]: the rank index is contiguous).
template <int DT, bool B_LAYOUT>
__global__ __launch_bounds__(256) void rowdot_kernel(const uint16_t *act, int64_t m, int64_t k,
                                                     int64_t ld, const uint16_t *w, int rank,
                                                     float scale, uint16_t *out) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= m) return;
    for (int j0 = 0; j0 < rank; j0 += 16) {
        float acc[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = 0.f;
        const int jn = rank - j0 < 16 ? rank - j0 : 16;
        for (int64_t c = lane * 8; c < k; c += 512) {
            float x[8];
            if (c + 8 <= k) {
                unpack8<DT>(*reinterpret_cast<const u32x4_t *>(act + row * ld + c), x);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = c + e < k ? ld1<DT>(act + row * ld + c + e) : 0.f;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                if (j >= jn) break;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (c + e < k) {
                        const uint16_t *wp = B_LAYOUT ? w + (c + e) * rank + j0 + j
                                                      : w + (j0 + j) * k + c + e;
                        acc[j] = fmaf(x[e], ld1<DT>(wp), acc[j]);
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (j >= jn) break;
            const float s = wave_sum(acc[j]);
            if (lane == 0) out[row * rank + j0 + j] = st1<DT>(s * scale);
        }
    }
}

// Partial sums over a chunk of rows: part[chunk][p][j] = sum_{m in chunk} U[m][p] * V[m][j].
template <int DT>
__global__ __launch_bounds__(256) void wgrad_partial_kernel(const uint16_t *u, int64_t m, int64_t p,
                                                            int64_t ldu, const uint16_t *v, int rank,
                                                            int64_t rows_per_chunk, float *part) {
    const int64_t col = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t chunk = blockIdx.y;
    const int64_t r0 = chunk * rows_per_chunk;
    const int64_t r1 = r0 + rows_per_chunk < m ? r0 + rows_per_chunk : m;
    for (int j0 = 0; j0 < rank; j0 += 16) {
        const int jn = rank - j0 < 16 ? rank - j0 : 16;
        float acc[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = 0.f;
        if (col < p) {
            for (int64_t r = r0; r < r1; ++r) {
                const float x = ld1<DT>(u + r * ldu + col);
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    if (j < jn) acc[j] = fmaf(x, ld1<DT>(v + r * rank + j0 + j), acc[j]);
            }
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (j < jn) part[(chunk * p + col) * rank + j0 + j] = acc[j];
        }
    }
}

__global__ __launch_bounds__(256) void wgrad_final_kernel(const float *part, int chunks, int64_t p,
                                                          int rank, float scale, float *out,
                                                          int transpose_out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= p * rank) return;
    float s = 0.f;
    for (int c = 0; c < chunks; ++c) s += part[c * p * rank + i];
    const int64_t col = i / rank, j = i % rank;
    if (transpose_out) out[j * p + col] = s * scale;
    else out[i] = s * scale;
}

// Element i of a [rows, cols] grid stride loop; row-strided operands.
template <int DT>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const uint16_t *gate, const uint16_t *up,
                                                         int64_t ld_gu, uint16_t *out, int64_t ld_h,
                                                         int64_t rows, int64_t cols) {
    const int64_t n = rows * cols;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t r = i / cols, c = i % cols;
        const float g = ld1<DT>(gate + r * ld_gu + c), u = ld1<DT>(up + r * ld_gu + c);
        const float sig = 1.0f / (1.0f + __expf(-g));
        out[r * ld_h + c] = st1<DT>(g * sig * u);
    }
}

template <int DT>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const uint16_t *grad, int64_t ld_h,
                                                         const uint16_t *gate, const uint16_t *up,
                                                         int64_t ld_gu, uint16_t *dgate,
                                                         uint16_t *dup, int64_t rows, int64_t cols) {
    const int64_t n = rows * cols;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t r = i / cols, c = i % cols;
        const float d = ld1<DT>(grad + r * ld_h + c);
        const float g = ld1<DT>(gate + r * ld_gu + c), u = ld1<DT>(up + r * ld_gu + c);
        const float sig = 1.0f / (1.0f + __expf(-g));
        // read both operands before either write: dgate/dup may alias gate/up
        const float vu = d * g * sig;
        const float vg = d * u * sig * (1.0f + g * (1.0f - sig));
        dup[r * ld_gu + c] = st1<DT>(vu);
        dgate[r * ld_gu + c] = st1<DT>(vg);
    }
}

// Column sums of dY, two passes like the LoRA weight gradients (rank 1, V = 1).
template <int DT>
__global__ __launch_bounds__(256) void colsum_partial_kernel(const uint16_t *dy, int64_t m, int64_t n,
                                                             int64_t ld, int64_t rows_per_chunk,
                                                             float *part) {
    const int64_t col = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * rows_per_chunk;
    const int64_t r1 = r0 + rows_per_chunk < m ? r0 + rows_per_chunk : m;
    if (col >= n) return;
    float s = 0.f;
    for (int64_t r = r0; r < r1; ++r) s += ld1<DT>(dy + r * ld + col);
    part[blockIdx.y * n + col] = s;
}

__global__ __launch_bounds__(256) void zero_kernel(float *out, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        out[i] = 0.f;
}

int grid_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    return static_cast<int>(b > 16384 ? 16384 : (b < 1 ? 1 : b));
}

constexpr int64_t kRowsPerChunk = 64;

}  // namespace

extern "C" int nf4_abi_version(void) { return NF4_ABI_VERSION; }

extern "C" const char *nf4_status_string(int status) {
    switch (status) {
        case NF4_OK: return "ok";
        case NF4_ERR_ARG: return "invalid argument";
        case NF4_ERR_UNSUPPORTED: return "unsupported layout or shape";
        case NF4_ERR_LAUNCH: return "HIP launch error";
        case NF4_ERR_WORKSPACE: return "workspace too small";
        default: return "unknown status";
    }
}

extern "C" int nf4_lora_xa(const void *xd, int64_t m, int64_t k, int64_t ldx, const void *a,
                           int rank, void *t, int dtype, void *stream) {
    if ((dtype != NF4_F16 && dtype != NF4_BF16) || m < 0 || k < 0 || rank < 1 || rank > kMaxRank)
        return NF4_ERR_ARG;
    if (m == 0) return NF4_OK;
    if (!xd || !a || !t || ldx < k) return NF4_ERR_ARG;
    if (ldx % 8 || !aligned(xd, 16)) return NF4_ERR_UNSUPPORTED;
    const dim3 grid(static_cast<unsigned>((m + 3) / 4));
    auto s = static_cast<hipStream_t>(stream);
    auto A = static_cast<const uint16_t *>(xd);
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL((rowdot_kernel<NF4_BF16, false>), grid, dim3(256), 0, s, A, m, k, ldx,
                           static_cast<const uint16_t *>(a), rank, 1.0f, static_cast<uint16_t *>(t));
    else
        hipLaunchKernelGGL((rowdot_kernel<NF4_F16, false>), grid, dim3(256), 0, s, A, m, k, ldx,
                           static_cast<const uint16_t *>(a), rank, 1.0f, static_cast<uint16_t *>(t));
    return status_of(hipGetLastError());
}

extern "C" int nf4_lora_da(const void *dy, int64_t m, int64_t n, int64_t lddy, const void *b,
                           int rank, float scale, void *da, int dtype, void *stream) {
    if ((dtype != NF4_F16 && dtype != NF4_BF16) || m < 0 || n < 0 || rank < 1 || rank > kMaxRank)
        return NF4_ERR_ARG;
    if (m == 0) return NF4_OK;
    if (!dy || !b || !da || lddy < n) return NF4_ERR_ARG;
    if (lddy % 8 || !aligned(dy, 16)) return NF4_ERR_UNSUPPORTED;
    const dim3 grid(static_cast<unsigned>((m + 3) / 4));
    auto s = static_cast<hipStream_t>(stream);
    auto A = static_cast<const uint16_t *>(dy);
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL((rowdot_kernel<NF4_BF16, true>), grid, dim3(256), 0, s, A, m, n, lddy,
                           static_cast<const uint16_t *>(b), rank, scale, static_cast<uint16_t *>(da));
    else
        hipLaunchKernelGGL((rowdot_kernel<NF4_F16, true>), grid, dim3(256), 0, s, A, m, n, lddy,
                           static_cast<const uint16_t *>(b), rank, scale, static_cast<uint16_t *>(da));
    return status_of(hipGetLastError());
}

extern "C" size_t nf4_lora_wgrad_workspace(int64_t m, int64_t p, int rank) {
    if (m <= 0 || p <= 0 || rank <= 0) return 0;
    const int64_t chunks = (m + kRowsPerChunk - 1) / kRowsPerChunk;
    return static_cast<size_t>(chunks) * p * rank * sizeof(float);
}

extern "C" int nf4_lora_wgrad(const void *u, int64_t m, int64_t p, int64_t ldu, const void *v,
                              int rank, float scale, float *out, int transpose_out, int dtype,
                              void *workspace, size_t workspace_bytes, void *stream) {
    if ((dtype != NF4_F16 && dtype != NF4_BF16) || m < 0 || p < 0 || rank < 1 || rank > kMaxRank)
        return NF4_ERR_ARG;
    if (!out || (m > 0 && (!u || !v)) || ldu < p) return NF4_ERR_ARG;
    auto s = static_cast<hipStream_t>(stream);
    if (p == 0) return NF4_OK;
    if (m == 0) {  // a fill kernel, not a memset node, so the call may be graph-captured
        hipLaunchKernelGGL(zero_kernel, dim3(grid_for(p * rank)), dim3(256), 0, s, out, p * rank);
        return status_of(hipGetLastError());
    }
    const size_t need = nf4_lora_wgrad_workspace(m, p, rank);
    if (!workspace || workspace_bytes < need) return NF4_ERR_WORKSPACE;
    const int64_t chunks = (m + kRowsPerChunk - 1) / kRowsPerChunk;
    if (chunks > 65535) return NF4_ERR_UNSUPPORTED;
    float *part = static_cast<float *>(workspace);
    const dim3 grid(static_cast<unsigned>((p + 255) / 256), static_cast<unsigned>(chunks));
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL(wgrad_partial_kernel<NF4_BF16>, grid, dim3(256), 0, s,
                           static_cast<const uint16_t *>(u), m, p, ldu,
                           static_cast<const uint16_t *>(v), rank, kRowsPerChunk, part);
    else
        hipLaunchKernelGGL(wgrad_partial_kernel<NF4_F16>, grid, dim3(256), 0, s,
                           static_cast<const uint16_t *>(u), m, p, ldu,
                           static_cast<const uint16_t *>(v), rank, kRowsPerChunk, part);
    int st = status_of(hipGetLastError());
    if (st != NF4_OK) return st;
    hipLaunchKernelGGL(wgrad_final_kernel, dim3(static_cast<unsigned>((p * rank + 255) / 256)),
                       dim3(256), 0, s, part, static_cast<int>(chunks), p, rank, scale, out,
                       transpose_out);
    return status_of(hipGetLastError());
}

extern "C" int nf4_swiglu_fwd(const void *gate, const void *up, int64_t ld_gu, void *out,
                              int64_t ld_h, int64_t rows, int64_t cols, int dtype, void *stream) {
    if ((dtype != NF4_F16 && dtype != NF4_BF16) || rows < 0 || cols < 0) return NF4_ERR_ARG;
    const int64_t n = rows * cols;
    if (n == 0) return NF4_OK;
    if (!gate || !up || !out || ld_gu < cols || ld_h < cols) return NF4_ERR_ARG;
    auto s = static_cast<hipStream_t>(stream);
    auto g = static_cast<const uint16_t *>(gate);
    auto u = static_cast<const uint16_t *>(up);
    auto o = static_cast<uint16_t *>(out);
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL(swiglu_fwd_kernel<NF4_BF16>, dim3(grid_for(n)), dim3(256), 0, s, g, u,
                           ld_gu, o, ld_h, rows, cols);
    else
        hipLaunchKernelGGL(swiglu_fwd_kernel<NF4_F16>, dim3(grid_for(n)), dim3(256), 0, s, g, u,
                           ld_gu, o, ld_h, rows, cols);
    return status_of(hipGetLastError());
}

extern "C" int nf4_swiglu_bwd(const void *grad, int64_t ld_h, const void *gate, const void *up,
                              int64_t ld_gu, void *dgate, void *dup, int64_t rows, int64_t cols,
                              int dtype, void *stream) {
    if ((dtype != NF4_F16 && dtype != NF4_BF16) || rows < 0 || cols < 0) return NF4_ERR_ARG;
    const int64_t n = rows * cols;
    if (n == 0) return NF4_OK;
    if (!grad || !gate || !up || !dgate || !dup || ld_gu < cols || ld_h < cols) return NF4_ERR_ARG;
    auto s = static_cast<hipStream_t>(stream);
    auto d = static_cast<const uint16_t *>(grad);
    auto g = static_cast<const uint16_t *>(gate);
    auto u = static_cast<const uint16_t *>(up);
    auto dg = static_cast<uint16_t *>(dgate);
    auto du = static_cast<uint16_t *>(dup);
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL(swiglu_bwd_kernel<NF4_BF16>, dim3(grid_for(n)), dim3(256), 0, s, d, ld_h,
                           g, u, ld_gu, dg, du, rows, cols);
    else
        hipLaunchKernelGGL(swiglu_bwd_kernel<NF4_F16>, dim3(grid_for(n)), dim3(256), 0, s, d, ld_h,
                           g, u, ld_gu, dg, du, rows, cols);
    return status_of(hipGetLastError());
}

extern "C" int nf4_bias_grad(const void *dy, int64_t m, int64_t n, int64_t lddy, float *out,
                             int dtype, void *stream) {
    if ((dtype != NF4_F16 && dtype != NF4_BF16) || m < 0 || n < 0 || !out) return NF4_ERR_ARG;
    auto s = static_cast<hipStream_t>(stream);
    if (n == 0) return NF4_OK;
    if (m == 0) {
        hipLaunchKernelGGL(zero_kernel, dim3(grid_for(n)), dim3(256), 0, s, out, n);
        return status_of(hipGetLastError());
    }
    if (!dy || lddy < n) return NF4_ERR_ARG;
    // One pass with a single chunk per column keeps this workspace-free: a thread per column,
    // rows in order (deterministic).
    const dim3 grid(static_cast<unsigned>((n + 255) / 256), 1);
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL(colsum_partial_kernel<NF4_BF16>, grid, dim3(256), 0, s,
                           static_cast<const uint16_t *>(dy), m, n, lddy, m, out);
    else
        hipLaunchKernelGGL(colsum_partial_kernel<NF4_F16>, grid, dim3(256), 0, s,
                           static_cast<const uint16_t *>(dy), m, n, lddy, m, out);
    return status_of(hipGetLastError());
}
