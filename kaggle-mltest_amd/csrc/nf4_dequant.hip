// Standalone NF4 dequantization for gfx950: packed 4-bit codes + double-quantized absmax ->
// fp16 / bf16 / fp32 weight, bit-exact with the reference's element formula
// (/root/reference/solution/nf4.py:26-55; layer.py:45-73).
//
// HBM-bound.  A thread owns "units" of 4 packed bytes = 8 elements: one 4-byte load, one absmax
// (blocksize is a multiple of 8), one 16-byte store (two for fp32).  Consecutive threads take
// consecutive units, so each wave reads 256 contiguous bytes and writes 1 KB contiguous per
// instruction; kUnroll independent units per thread, all loaded before any wait, keep loads in
// flight.  The NF4 table and the 256-entry absmax code map sit in LDS.  The absmax is rebuilt
// per unit from its uint8 code, never materialised in HBM.

#include "nf4_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;

struct DequantArgs {
    DevWeight w[NF4_MAX_SEGMENTS];
    void *out[NF4_MAX_SEGMENTS];           // each segment's [rows, cols] output
    int64_t block_start[NF4_MAX_SEGMENTS + 1];
    int nseg;
};

// 8 consecutive outputs, streamed (non-temporal: the weight is written once, read later by
// another kernel).
template <int DT>
__device__ __forceinline__ void store8(void *out, int64_t e, const float (&v)[8]) {
    if constexpr (DT == NF4_F32) {
        float4_t *o = reinterpret_cast<float4_t *>(static_cast<float *>(out) + e);
        __builtin_nontemporal_store((float4_t){v[0], v[1], v[2], v[3]}, o);
        __builtin_nontemporal_store((float4_t){v[4], v[5], v[6], v[7]}, o + 1);
    } else {
        u32x4_t r;
        r.x = pack2<DT>(v[0], v[1]);
        r.y = pack2<DT>(v[2], v[3]);
        r.z = pack2<DT>(v[4], v[5]);
        r.w = pack2<DT>(v[6], v[7]);
        __builtin_nontemporal_store(r, reinterpret_cast<u32x4_t *>(static_cast<uint16_t *>(out) + e));
    }
}

template <int DT>
__device__ __forceinline__ void store1(void *out, int64_t e, float v) {
    if constexpr (DT == NF4_F32) {
        static_cast<float *>(out)[e] = v;
    } else {
        static_cast<uint16_t *>(out)[e] = round16<DT>(v);
    }
}

__device__ __forceinline__ int find_segment(const DequantArgs &a, int64_t blk) {
    int s = 0;
#pragma unroll
    for (int i = 1; i < NF4_MAX_SEGMENTS; ++i)
        if (i < a.nseg && blk >= a.block_start[i]) s = i;
    return s;
}

// Fast path: every segment has a power-of-two blocksize >= 8 (and absmax group when nested), a
// 4-byte aligned packed pointer, a 16-byte aligned output start and fewer than 2^32 elements.
// All loads of a thread (packed units, uint8 absmax codes, absmax2 scales) are issued first,
// through buffer resources (past the end reads zero, so they need no branches), then the
// tables; one wait covers them all.  Elements past the last full unit are done one by one.
template <int DT>
__global__ __launch_bounds__(kThreads) void dequant_units_kernel(const DequantArgs a) {
    __shared__ float s_code[16];
    __shared__ float s_code2[256];
    const int seg = find_segment(a, blockIdx.x);
    const DevWeight &w = a.w[seg];
    const int64_t n = w.rows * w.cols;
    const int64_t units = n >> 3;
    const int64_t nb = (n + w.blocksize - 1) >> w.bs_shift;
    const int64_t lb = static_cast<int64_t>(blockIdx.x) - a.block_start[seg];
    const rsrc_t pk = make_rsrc(w.packed, units * 4);
    const rsrc_t qr = make_rsrc(w.absmax, w.nested ? nb : nb * 4);
    const rsrc_t sr = w.nested ? make_rsrc(w.absmax2, ((nb + w.blocksize2 - 1) >> w.bs2_shift) * 4)
                               : qr;

    uint32_t p[kUnroll], q[kUnroll];
    float sc[kUnroll];
    const uint32_t u0 = static_cast<uint32_t>(lb * (kUnroll * kThreads)) + threadIdx.x;
#pragma unroll
    for (int g = 0; g < kUnroll; ++g) {
        const uint32_t u = u0 + g * kThreads;
        p[g] = bload4(pk, static_cast<int>(u * 4));
        const uint32_t b = (u << 3) >> w.bs_shift;
        if (w.nested) {
            q[g] = bload1(qr, static_cast<int>(b));
            sc[g] = __builtin_bit_cast(float, bload4(sr, static_cast<int>((b >> w.bs2_shift) * 4)));
        } else {
            q[g] = 0;
            sc[g] = __builtin_bit_cast(float, bload4(qr, static_cast<int>(b * 4)));
        }
    }
    if (threadIdx.x < 16) s_code[threadIdx.x] = w.code[threadIdx.x];
    if (w.nested) s_code2[threadIdx.x] = w.code2[threadIdx.x];
    __syncthreads();

    void *out = a.out[seg];
    const int64_t off = 0;
#pragma unroll
    for (int g = 0; g < kUnroll; ++g) {
        const int64_t u = u0 + g * kThreads;
        if (u < units) {
            const float s = w.nested ? __fadd_rn(__fmul_rn(s_code2[q[g]], sc[g]), w.offset) : sc[g];
            float v[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[2 * j] = __fmul_rn(s_code[(p[g] >> (8 * j + 4)) & 0xF], s);
                v[2 * j + 1] = __fmul_rn(s_code[(p[g] >> (8 * j)) & 0xF], s);
            }
            store8<DT>(out, off + (u << 3), v);
        } else if (u == units && (n & 7)) {
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
        store1<DT>(a.out[seg], e, __fmul_rn(s_code[nib], s));
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


// Shared by the stacked and batched entry points: segment i goes to outs[i].
int dequant_segments(const nf4_weight *ws, int nw, void *const *outs, int out_dtype,
                     void *stream) {
    DequantArgs a = {};
    a.nseg = nw;
    bool units_ok = true;
    for (int i = 0; i < nw; ++i) {
        const int st = check_weight(&ws[i]);
        if (st != NF4_OK) return st;
        a.w[i] = to_dev(ws[i]);
        a.out[i] = outs[i];
        const int64_t n = ws[i].rows * ws[i].cols;
        if (n > 0 && !outs[i]) return NF4_ERR_ARG;
        units_ok = units_ok && ws[i].blocksize >= 8 && log2_exact(ws[i].blocksize) >= 0 &&
                   (!ws[i].nested || log2_exact(ws[i].blocksize2) >= 0) &&
                   aligned(ws[i].packed, 4) && aligned(outs[i], 16) && n < (int64_t(1) << 32);
    }
    const int path = units_ok ? kUnits : kElements;
    // Grid: the vector path covers ceil(units (+1 partial) / (threads * unroll)) workgroups per
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

}  // namespace

extern "C" int nf4_dequant_multi(const nf4_weight *ws, int nw, void *out, int out_dtype,
                                 void *stream) {
    if (!ws || nw < 1 || nw > NF4_MAX_SEGMENTS) return NF4_ERR_ARG;
    if (out_dtype != NF4_F16 && out_dtype != NF4_BF16 && out_dtype != NF4_F32) return NF4_ERR_ARG;
    int64_t total = 0;
    for (int i = 0; i < nw; ++i) total += ws[i].rows * ws[i].cols;
    if (total == 0) return NF4_OK;  // nothing to write (out may be null)
    if (!out) return NF4_ERR_ARG;
    void *outs[NF4_MAX_SEGMENTS];
    int64_t off = 0;
    for (int i = 0; i < nw; ++i) {
        if (ws[i].cols != ws[0].cols) return NF4_ERR_ARG;
        outs[i] = static_cast<char *>(out) + off * dtype_bytes(out_dtype);
        off += ws[i].rows * ws[i].cols;
    }
    return dequant_segments(ws, nw, outs, out_dtype, stream);
}

extern "C" int nf4_dequant_batch(const nf4_weight *ws, int nw, void *const *outs, int out_dtype,
                                 void *stream) {
    if (!ws || !outs || nw < 1 || nw > NF4_MAX_SEGMENTS) return NF4_ERR_ARG;
    if (out_dtype != NF4_F16 && out_dtype != NF4_BF16 && out_dtype != NF4_F32) return NF4_ERR_ARG;
    int64_t total = 0;
    for (int i = 0; i < nw; ++i) total += ws[i].rows * ws[i].cols;
    if (total == 0) return NF4_OK;
    return dequant_segments(ws, nw, outs, out_dtype, stream);
}

extern "C" int nf4_dequant(const nf4_weight *w, void *out, int out_dtype, void *stream) {
    return nf4_dequant_multi(w, 1, out, out_dtype, stream);
}
