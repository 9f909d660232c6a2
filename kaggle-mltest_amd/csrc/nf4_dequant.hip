// Standalone NF4 dequantization for gfx950: packed 4-bit codes + double-quantized absmax ->
// fp16 / bf16 / fp32 weight, bit-exact with the reference's element formula
// (/root/reference/solution/nf4.py:26-55; layer.py:45-73).
//
// HBM-bound.  A thread owns "units" of 4 packed bytes = 8 elements: one 4-byte load, one absmax
// (blocksize is a multiple of 8), one 16-byte store (two for fp32).  Consecutive threads take
// consecutive units, so each wave reads 256 contiguous bytes and writes 1 KB contiguous per
// instruction; UNROLL independent units per thread keep loads in flight.  The NF4 table and the
// 256-entry absmax code map sit in LDS.  The absmax is rebuilt per unit from its uint8 code,
// never materialised in HBM.

#include "nf4_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

struct DequantArgs {
    DevWeight w[NF4_MAX_SEGMENTS];
    int64_t out_off[NF4_MAX_SEGMENTS];     // element offset of each segment in `out`
    int64_t block_start[NF4_MAX_SEGMENTS + 1];
    int nseg;
    void *out;
};

template <int DT>
__device__ __forceinline__ void store8(void *out, int64_t e, const float (&v)[8]) {
    if constexpr (DT == NF4_F32) {
        float4_t *o = reinterpret_cast<float4_t *>(static_cast<float *>(out) + e);
        o[0] = (float4_t){v[0], v[1], v[2], v[3]};
        o[1] = (float4_t){v[4], v[5], v[6], v[7]};
    } else {
        u32x4_t r;
        r.x = pack2<DT>(v[0], v[1]);
        r.y = pack2<DT>(v[2], v[3]);
        r.z = pack2<DT>(v[4], v[5]);
        r.w = pack2<DT>(v[6], v[7]);
        *reinterpret_cast<u32x4_t *>(static_cast<uint16_t *>(out) + e) = r;
    }
}

template <int DT>
__device__ __forceinline__ void store1(void *out, int64_t e, float v) {
    if constexpr (DT == NF4_F32) {
        static_cast<float *>(out)[e] = v;
    } else if constexpr (DT == NF4_BF16) {
        static_cast<bf16_t *>(out)[e] = static_cast<bf16_t>(v);
    } else {
        static_cast<half_t *>(out)[e] = static_cast<half_t>(v);
    }
}

__device__ __forceinline__ int find_segment(const DequantArgs &a, int64_t blk) {
    int s = 0;
#pragma unroll
    for (int i = 1; i < NF4_MAX_SEGMENTS; ++i)
        if (i < a.nseg && blk >= a.block_start[i]) s = i;
    return s;
}

// Fast path: every segment has blocksize % 8 == 0, a 4-byte aligned packed pointer and a
// 16-byte aligned output start.  Elements past the last full unit are done one by one.
template <int DT>
__global__ __launch_bounds__(kThreads) void dequant_units_kernel(const DequantArgs a) {
    __shared__ float s_code[16];
    __shared__ float s_code2[256];
    const int seg = find_segment(a, blockIdx.x);
    const DevWeight &w = a.w[seg];
    if (threadIdx.x < 16) s_code[threadIdx.x] = w.code[threadIdx.x];
    if (w.nested) s_code2[threadIdx.x] = w.code2[threadIdx.x];
    __syncthreads();

    const int64_t n = w.rows * w.cols;
    const int64_t units = n >> 3;
    void *out = a.out;
    const int64_t off = a.out_off[seg];
    const int64_t lb = static_cast<int64_t>(blockIdx.x) - a.block_start[seg];
    const uint32_t *packed32 = reinterpret_cast<const uint32_t *>(w.packed);

    uint32_t p[kUnroll];
    int64_t u[kUnroll];
#pragma unroll
    for (int g = 0; g < kUnroll; ++g) {
        u[g] = (lb * kUnroll + g) * kThreads + threadIdx.x;
        p[g] = u[g] < units ? __builtin_nontemporal_load(packed32 + u[g]) : 0u;
    }
#pragma unroll
    for (int g = 0; g < kUnroll; ++g) {
        if (u[g] < units) {
            const float s = absmax_of(w, s_code2, block_index(w, u[g] << 3));
            float v[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[2 * j] = __fmul_rn(s_code[(p[g] >> (8 * j + 4)) & 0xF], s);
                v[2 * j + 1] = __fmul_rn(s_code[(p[g] >> (8 * j)) & 0xF], s);
            }
            store8<DT>(out, off + (u[g] << 3), v);
        } else if (u[g] == units && (n & 7)) {
            for (int64_t e = units << 3; e < n; ++e) {
                const uint8_t byte = w.packed[e >> 1];
                const int nib = (e & 1) ? (byte & 0xF) : (byte >> 4);
                const float s = absmax_of(w, s_code2, block_index(w, e));
                store1<DT>(out, off + e, __fmul_rn(s_code[nib], s));
            }
        }
    }
}

// General path (any even blocksize, any alignment): one element per thread, grid-stride.
template <int DT>
__global__ __launch_bounds__(kThreads) void dequant_elements_kernel(const DequantArgs a) {
    __shared__ float s_code[16];
    __shared__ float s_code2[256];
    const int seg = find_segment(a, blockIdx.x);
    const DevWeight &w = a.w[seg];
    if (threadIdx.x < 16) s_code[threadIdx.x] = w.code[threadIdx.x];
    if (w.nested) s_code2[threadIdx.x] = w.code2[threadIdx.x];
    __syncthreads();
    const int64_t n = w.rows * w.cols;
    const int64_t lb = static_cast<int64_t>(blockIdx.x) - a.block_start[seg];
    const int64_t nblocks = a.block_start[seg + 1] - a.block_start[seg];
    for (int64_t e = lb * kThreads + threadIdx.x; e < n; e += nblocks * kThreads) {
        const uint8_t byte = w.packed[e >> 1];
        const int nib = (e & 1) ? (byte & 0xF) : (byte >> 4);
        const float s = absmax_of(w, s_code2, block_index(w, e));
        store1<DT>(a.out, a.out_off[seg] + e, __fmul_rn(s_code[nib], s));
    }
}

enum Path { kElements = 0, kUnits = 1 };

template <int DT>
void launch_dt(const DequantArgs &a, int path, dim3 g, hipStream_t stream) {
    const dim3 b(kThreads);
    if (path == kUnits) hipLaunchKernelGGL(dequant_units_kernel<DT>, g, b, 0, stream, a);
    else hipLaunchKernelGGL(dequant_elements_kernel<DT>, g, b, 0, stream, a);
}

int launch(DequantArgs &a, int path, int dt, hipStream_t stream) {
    const int64_t grid = a.block_start[a.nseg];
    if (grid == 0) return NF4_OK;
    if (grid > 0x7fffffff) return NF4_ERR_UNSUPPORTED;
    const dim3 g(static_cast<unsigned>(grid));
    if (dt == NF4_F16) launch_dt<NF4_F16>(a, path, g, stream);
    else if (dt == NF4_BF16) launch_dt<NF4_BF16>(a, path, g, stream);
    else launch_dt<NF4_F32>(a, path, g, stream);
    return status_of(hipGetLastError());
}

}  // namespace

extern "C" int nf4_dequant_multi(const nf4_weight *ws, int nw, void *out, int out_dtype,
                                 void *stream) {
    if (!ws || nw < 1 || nw > NF4_MAX_SEGMENTS) return NF4_ERR_ARG;
    if (out_dtype != NF4_F16 && out_dtype != NF4_BF16 && out_dtype != NF4_F32) return NF4_ERR_ARG;
    int64_t total = 0;
    for (int i = 0; i < nw; ++i) total += ws[i].rows * ws[i].cols;
    if (total == 0) return NF4_OK;  // nothing to write (out may be null)
    if (!out) return NF4_ERR_ARG;
    const int dts = dtype_bytes(out_dtype);
    DequantArgs a = {};
    a.nseg = nw;
    a.out = out;
    int64_t off = 0;
    bool units_ok = aligned(out, 16);
    for (int i = 0; i < nw; ++i) {
        const int st = check_weight(&ws[i]);
        if (st != NF4_OK) return st;
        if (ws[i].cols != ws[0].cols) return NF4_ERR_ARG;
        a.w[i] = to_dev(ws[i]);
        a.out_off[i] = off;
        const int64_t n = ws[i].rows * ws[i].cols;
        const bool out_ok = (off * dts) % 16 == 0;
        units_ok = units_ok && (ws[i].blocksize % 8 == 0) && aligned(ws[i].packed, 4) && out_ok;
        off += n;
    }
    const int path = units_ok ? kUnits : kElements;
    // Grid: the vector paths cover ceil(units (+1 partial) / (threads * unroll)) workgroups per
    // segment; the general path a bounded grid-stride grid.
    a.block_start[0] = 0;
    for (int i = 0; i < nw; ++i) {
        const int64_t n = ws[i].rows * ws[i].cols;
        int64_t blocks;
        if (path == kUnits) {
            const int64_t units = (n >> 3) + ((n & 7) ? 1 : 0);
            blocks = (units + kThreads * kUnroll - 1) / (kThreads * kUnroll);
        } else {
            blocks = (n + kThreads - 1) / kThreads;
            if (blocks > 65536) blocks = 65536;
        }
        a.block_start[i + 1] = a.block_start[i] + blocks;
    }
    return launch(a, path, out_dtype, static_cast<hipStream_t>(stream));
}

extern "C" int nf4_dequant(const nf4_weight *w, void *out, int out_dtype, void *stream) {
    return nf4_dequant_multi(w, 1, out, out_dtype, stream);
}
