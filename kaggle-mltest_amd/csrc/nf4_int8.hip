// int8 input-gradient path of the MLP on gfx950 (the reference's T4 int8 backward,
// /root/reference/solution/layer.py:299-442, 515-618, 992-1013), kept off the fp16 parity path:
//   - column scales of a stack of NF4 weights (largest |W| per input column, W rounded to the
//     GEMM dtype) and the stack as int8 transposed with those scales, or as int8 rows with
//     one scale per row;
//   - one int8 row per activation row (scale = largest |x| / 127);
//   - C = A . B^T over int8 operands on v_mfma_i32_32x32x32_i8 with exact int32 sums, written as
//     int32 or scaled to fp16 / bf16 (split-K partials are int32 too, so any split order gives
//     the same sums);
//   - SwiGLU backward on the int32 sums of the down projection's input gradient with per-row
//     int8 requantization of both halves.
// Rounding: ties away from zero, clamped to [-127, 127] (layer.py:299-303); every fp32 product,
// quotient and sum rounded on its own (no contraction).
#include "nf4_common.h"

namespace {

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef int v16i_t __attribute__((ext_vector_type(16)));

constexpr int kSegs = NF4_MAX_SEGMENTS;

__device__ __forceinline__ int round_i8(float v) {
    const float r = v >= 0.0f ? floorf(__fadd_rn(v, 0.5f)) : -floorf(__fsub_rn(0.5f, v));
    return static_cast<int>(fminf(fmaxf(r, -127.0f), 127.0f));
}

template <int DT>
__device__ __forceinline__ float load_act(const uint16_t *p) {
    if constexpr (DT == NF4_BF16) return static_cast<float>(__builtin_bit_cast(bf16_t, *p));
    else return static_cast<float>(__builtin_bit_cast(half_t, *p));
}

// |value rounded to the GEMM dtype| as its magnitude bits (monotonic in the value).
template <int DT>
__device__ __forceinline__ uint32_t mag_bits(float v) {
    return round16<DT>(v) & 0x7fffu;
}

template <int DT>
__device__ __forceinline__ float from_mag(uint32_t m) {
    if constexpr (DT == NF4_BF16) return static_cast<float>(__builtin_bit_cast(bf16_t, static_cast<uint16_t>(m)));
    else return static_cast<float>(__builtin_bit_cast(half_t, static_cast<uint16_t>(m)));
}

// Block-wide reductions over 256 threads (4 waves): wave shuffles, then the 4 wave values
// through LDS in wave order.
__device__ __forceinline__ float block_max(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Stacked weights: segment descriptors plus the first stacked row of each.
struct StackArgs {
    DevWeight w[kSegs];
    int64_t row0[kSegs + 1];  // cumulative rows
    int64_t tile0[kSegs + 1]; // cumulative 64-row (or 256-row) tiles
    int nseg;
    int64_t cols;
};

__device__ __forceinline__ int seg_of(const StackArgs &a, int64_t t) {
    int s = 0;
#pragma unroll
    for (int i = 1; i < kSegs; ++i)
        if (i < a.nseg && t >= a.tile0[i]) s = i;
    return s;
}

__device__ __forceinline__ void fill_tables(const DevWeight &w, float *code2, float *code) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x)
        code2[i] = w.nested ? w.code2[i] : 0.0f;
    if (threadIdx.x < 16) code[threadIdx.x] = w.code[threadIdx.x];
    __syncthreads();
}

// fp32 dequantized element e of weight w (bitsandbytes' value before the rounding to a dtype).
__device__ __forceinline__ float nf4_value(const DevWeight &w, const float *code2, const float *code,
                                          int64_t e) {
    const uint8_t byte = w.packed[e >> 1];
    const int nib = (e & 1) ? (byte & 15) : (byte >> 4);
    return __fmul_rn(code[nib], absmax_of(w, code2, block_index(w, e)));
}

// ---------------------------------------------------------------------- column scales

// Partial column maxima: workgroup (x, y) takes columns 256x .. 256x+255 over the 256-row tile y
// of the stack (tiles numbered segment by segment), writing |W| magnitude bits per column.
template <int DT>
__global__ __launch_bounds__(256) void colmax_partial_kernel(const StackArgs a, uint16_t *part) {
    __shared__ float s_code2[256];
    __shared__ float s_code[16];
    const int64_t t = blockIdx.y;
    const int seg = seg_of(a, t);
    const DevWeight &w = a.w[seg];
    fill_tables(w, s_code2, s_code);
    const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (c >= a.cols) return;
    const int64_t r0 = (t - a.tile0[seg]) * 256;
    const int64_t r1 = r0 + 256 < w.rows ? r0 + 256 : w.rows;
    uint32_t m = 0;
#pragma unroll 8
    for (int64_t r = r0; r < r1; ++r) {
        const uint32_t b = mag_bits<DT>(nf4_value(w, s_code2, s_code, r * a.cols + c));
        m = b > m ? b : m;
    }
    part[t * a.cols + c] = static_cast<uint16_t>(m);
}

// scale[c] = max(largest |W[:, c]|, 1e-20) / 127 from the partial maxima of every row tile.
template <int DT>
__global__ __launch_bounds__(256) void colmax_final_kernel(const uint16_t *part, int64_t tiles,
                                                           int64_t cols, float *scale) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (c >= cols) return;
    uint32_t m = 0;
    for (int64_t t = 0; t < tiles; ++t) {
        const uint32_t b = part[t * cols + c];
        m = b > m ? b : m;
    }
    scale[c] = __fdiv_rn(fmaxf(from_mag<DT>(m), 1e-20f), 127.0f);
}

// ------------------------------------------------------------------- int8 weights

// The stack transposed: workgroup = 64 rows x 64 columns of one segment; q[c][row0 + r] =
// round(W[r][c] / scale[c]) through an LDS tile (64 x 64 bytes, rows padded to 80 bytes).
__global__ __launch_bounds__(256) void int8_weight_t_kernel(const StackArgs a, const float *scale,
                                                            int8_t *q, int64_t ldq) {
    __shared__ float s_code2[256];
    __shared__ float s_code[16];
    __shared__ __attribute__((aligned(16))) int8_t tile[64][80];
    const int64_t t = blockIdx.y;
    const int seg = seg_of(a, t);
    const DevWeight &w = a.w[seg];
    fill_tables(w, s_code2, s_code);
    const int64_t r0 = (t - a.tile0[seg]) * 64;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int rl = threadIdx.x >> 2, cq = (threadIdx.x & 3) * 16;
    {
        const int64_t e0 = (r0 + rl) * a.cols + c0 + cq;  // 16 elements inside one absmax block
        const uint2 raw = *reinterpret_cast<const uint2 *>(w.packed + (e0 >> 1));
        const float am = absmax_of(w, s_code2, block_index(w, e0));
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t word = i < 8 ? raw.x : raw.y;
            const int byte = (word >> (8 * ((i & 7) >> 1))) & 0xff;
            const int nib = (i & 1) ? (byte & 15) : (byte >> 4);
            const float v = __fmul_rn(s_code[nib], am);
            tile[cq + i][rl] = static_cast<int8_t>(round_i8(__fdiv_rn(v, scale[c0 + cq + i])));
        }
    }
    __syncthreads();
    // write: thread -> output row c0 + cl, 16 stacked rows starting at row0 + r0 + rq
    const int cl = threadIdx.x >> 2, rq = (threadIdx.x & 3) * 16;
    int8_t *dst = q + (c0 + cl) * ldq + a.row0[seg] + r0 + rq;
    *reinterpret_cast<u32x4_t *>(dst) = *reinterpret_cast<const u32x4_t *>(&tile[cl][rq]);
}

// The stack as int8 rows: one workgroup per stacked row r, s[r] = max(largest |W[r]|, 1e-20) /
// 127, q[r][c] = round(W[r][c] * (127 / largest)) with W the fp32 dequantized value
// (layer.py:306-335).
__global__ __launch_bounds__(256) void int8_weight_rows_kernel(const StackArgs a, int8_t *q,
                                                               int64_t ldq, float *s) {
    __shared__ float s_code2[256];
    __shared__ float s_code[16];
    __shared__ float red[4];
    const int64_t r = blockIdx.x;
    int seg = 0;
#pragma unroll
    for (int i = 1; i < kSegs; ++i)
        if (i < a.nseg && r >= a.row0[i]) seg = i;
    const DevWeight &w = a.w[seg];
    fill_tables(w, s_code2, s_code);
    const int64_t lr = r - a.row0[seg];
    float top = 0.0f;
    for (int64_t c = threadIdx.x; c < a.cols; c += 256)
        top = fmaxf(top, fabsf(nf4_value(w, s_code2, s_code, lr * a.cols + c)));
    top = fmaxf(block_max(top, red), 1e-20f);
    const float inv = __fdiv_rn(127.0f, top);
    for (int64_t c = threadIdx.x; c < a.cols; c += 256)
        q[r * ldq + c] = static_cast<int8_t>(
            round_i8(__fmul_rn(nf4_value(w, s_code2, s_code, lr * a.cols + c), inv)));
    if (threadIdx.x == 0) s[r] = __fdiv_rn(top, 127.0f);
}

// ------------------------------------------------------------------- int8 activations

// 8 consecutive elements of a row (fp16 / bf16: one 16-byte load; fp32: two) as fp32.
template <int DT>
__device__ __forceinline__ void load8(const void *p, float (&v)[8]) {
    if constexpr (DT == NF4_F32) {
        const float4_t a = reinterpret_cast<const float4_t *>(p)[0];
        const float4_t b = reinterpret_cast<const float4_t *>(p)[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = a[i];
            v[4 + i] = b[i];
        }
    } else {
        const u32x4_t w = *reinterpret_cast<const u32x4_t *>(p);
        const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint16_t lo = wv[i] & 0xffff, hi = wv[i] >> 16;
            v[2 * i] = load_act<DT>(&lo);
            v[2 * i + 1] = load_act<DT>(&hi);
        }
    }
}

// One int8 row per row of x (layer.py:372-382), 8 elements per thread access.
template <int DT>
__global__ __launch_bounds__(256) void int8_rows_kernel(const uint8_t *x, int64_t cols,
                                                        int64_t ldx_bytes, int8_t *q, int64_t ldq,
                                                        float *s) {
    constexpr int EB = DT == NF4_F32 ? 4 : 2;
    __shared__ float red[4];
    const int64_t r = blockIdx.x;
    const uint8_t *row = x + r * ldx_bytes;
    float top = 0.0f;
    for (int64_t c = threadIdx.x * 8; c < cols; c += 256 * 8) {
        float v[8];
        load8<DT>(row + c * EB, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) top = fmaxf(top, fabsf(v[i]));
    }
    top = fmaxf(block_max(top, red), 1e-20f);
    const float inv = __fdiv_rn(127.0f, top);
    for (int64_t c = threadIdx.x * 8; c < cols; c += 256 * 8) {
        float v[8];
        load8<DT>(row + c * EB, v);
        uint32_t o[2] = {0u, 0u};
#pragma unroll
        for (int i = 0; i < 8; ++i)
            o[i >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(round_i8(__fmul_rn(v[i], inv))))
                         << (8 * (i & 3));
        *reinterpret_cast<u32x2_t *>(q + r * ldq + c) = (u32x2_t){o[0], o[1]};
    }
    if (threadIdx.x == 0) s[r] = __fdiv_rn(top, 127.0f);
}

// ------------------------------------------------------------------------ int8 GEMM
//
// C[m][n] = sum_k A[m][k] B[n][k], 128 x 128 tiles, 4 waves of 64 x 64, 128-byte k steps.  Both
// operands are staged like the activation tile of the NF4 GEMMs (16-byte loads into registers
// two steps ahead, LDS rows of 128 bytes with 16-byte chunks XOR-swizzled by bits 1-3 of the
// row, the next step's LDS stores interleaved with the MFMAs).  The MFMA A operand is the B
// tile (rows n) and its B operand the A tile (rows m), so that a lane's four consecutive
// accumulator rows are four consecutive output columns.  A k-substep covers 32 bytes: lane l
// reads the 16 bytes of chunk 2 ks + l / 32 of its row in both operands (the same k order in
// both, as the product requires).
constexpr int IBR = 128;  // k bytes per step

struct I8Args {
    const int8_t *a;
    const int8_t *b;
    int64_t M, N, K, lda, ldb;
    const float *sa, *sb;
    void *c;
    int64_t ldc;
    int32_t *partial;  // split-K: [splits][M][N] int32
    int splits;
    int64_t per_split;
    int64_t m_tiles;
};

__device__ __forceinline__ int i8swz(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

template <int NT>
struct I8Tile {  // NT / 2 rows x 128 bytes, 4 chunks of 16 bytes per thread
    u32x4_t r[4];
    __device__ __forceinline__ void load(rsrc_t rs, int base, int rstep, int col) {
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = bload16(rs, base + i * rstep + col);
    }
    __device__ __forceinline__ void store_part(uint8_t *s, int part) const {
        const int idx = part * NT + threadIdx.x;
        *reinterpret_cast<u32x4_t *>(s + i8swz(idx >> 3, idx & 7)) = r[part];
    }
};

// BT x BT tiles: 128 (4 waves of 64 x 64, two workgroups per CU) or 256 (8 waves of 128 n x
// 64 m, one per CU: half the LDS bytes per MFMA).
template <int EPI, int BT>  // EPI 0: int32 C (or split partials), 1: fp16 C, 2: bf16 C
__global__ __launch_bounds__(BT * 2) void i8_gemm_kernel(const I8Args g) {
    constexpr int NT = BT * 2, WN = 2, WM = NT / 64 / WN;
    constexpr int TN = BT / WN / 32, TM = BT / WM / 32;
    __shared__ __attribute__((aligned(1024))) uint8_t sA[2][BT * 128];
    __shared__ __attribute__((aligned(1024))) uint8_t sB[2][BT * 128];
    const uint32_t nsp = static_cast<uint32_t>(g.splits);
    const uint32_t blk = blockIdx.x;
    const uint32_t tile = __builtin_amdgcn_readfirstlane(blk / nsp);
    const int split = __builtin_amdgcn_readfirstlane(static_cast<int>(blk % nsp));
    const uint32_t mtl = static_cast<uint32_t>(g.m_tiles);
    const int64_t n0 = static_cast<int64_t>(__builtin_amdgcn_readfirstlane(tile / mtl)) * BT;
    const int64_t m0 = static_cast<int64_t>(__builtin_amdgcn_readfirstlane(tile % mtl)) * BT;
    const int64_t steps = g.K / IBR;
    const int64_t s0 = split * g.per_split;
    const int64_t s1 = s0 + g.per_split < steps ? s0 + g.per_split : steps;

    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int wn = wave % WN, wm = wave / WN;
    const int lane = threadIdx.x & 63, r = lane & 31, kh = lane >> 5;

    // windows: rows past M / N read as zero
    const int64_t ma = g.M - m0 < BT ? g.M - m0 : BT, nb = g.N - n0 < BT ? g.N - n0 : BT;
    const rsrc_t ra = make_rsrc(g.a + m0 * g.lda, (ma - 1) * g.lda + g.K);
    const rsrc_t rb = make_rsrc(g.b + n0 * g.ldb, (nb - 1) * g.ldb + g.K);
    const int t = threadIdx.x;
    const int abase = static_cast<int>((t >> 3) * g.lda + (t & 7) * 16);
    const int bbase = static_cast<int>((t >> 3) * g.ldb + (t & 7) * 16);
    const int astep = static_cast<int>((NT / 8) * g.lda), bstep = static_cast<int>((NT / 8) * g.ldb);

    v16i_t acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = (v16i_t){};

    auto mma = [&](int b, auto &&part) {
#pragma unroll
        for (int ks = 0; ks < IBR / 32; ++ks) {
            const int c = ks * 2 + kh;
            v4i_t fn[TN], fm[TM];
#pragma unroll
            for (int i = 0; i < TN; ++i)
                fn[i] = *reinterpret_cast<const v4i_t *>(sB[b] + i8swz(wn * (BT / WN) + i * 32 + r, c));
#pragma unroll
            for (int j = 0; j < TM; ++j)
                fm[j] = *reinterpret_cast<const v4i_t *>(sA[b] + i8swz(wm * (BT / WM) + j * 32 + r, c));
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fn[i], fm[j], acc[i][j], 0, 0, 0);
            part(ks);
        }
    };

    I8Tile<NT> ta[2], tb[2];
    if (s0 < s1) {
        ta[0].load(ra, abase, astep, static_cast<int>(s0) * IBR);
        tb[0].load(rb, bbase, bstep, static_cast<int>(s0) * IBR);
        ta[1].load(ra, abase, astep, static_cast<int>(s0 + 1) * IBR);
        tb[1].load(rb, bbase, bstep, static_cast<int>(s0 + 1) * IBR);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            ta[0].store_part(sA[0], q);
            tb[0].store_part(sB[0], q);
        }
        __syncthreads();
        int64_t st = s0;
        for (; st + 1 < s1; st += 2) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                ta[b].load(ra, abase, astep, static_cast<int>(st + b + 2) * IBR);
                tb[b].load(rb, bbase, bstep, static_cast<int>(st + b + 2) * IBR);
                mma(b, [&](int ks) {
                    ta[b ^ 1].store_part(sA[b ^ 1], ks);
                    tb[b ^ 1].store_part(sB[b ^ 1], ks);
                });
                __syncthreads();
            }
        }
        if (st < s1) mma(0, [](int) {});
    }

    // epilogue: lane holds C[m][n .. n+3] for m = m0 + wm BT/WM + j 32 + r,
    // n = n0 + wn BT/WN + i 32 + 8 r4 + 4 kh
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const int64_t m = m0 + wm * (BT / WM) + j * 32 + r;
        if (m >= g.M) continue;
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int64_t n = n0 + wn * (BT / WN) + i * 32 + r4 * 8 + kh * 4;
                if (n >= g.N) continue;
                const int v[4] = {acc[i][j][4 * r4], acc[i][j][4 * r4 + 1], acc[i][j][4 * r4 + 2],
                                  acc[i][j][4 * r4 + 3]};
                const bool full = n + 4 <= g.N;
                if (EPI == 0 || g.splits > 1) {
                    int32_t *dst = g.splits > 1
                                       ? g.partial + (static_cast<int64_t>(split) * g.M + m) * g.N + n
                                       : static_cast<int32_t *>(g.c) + m * g.ldc + n;
                    if (full) *reinterpret_cast<v4i_t *>(dst) = (v4i_t){v[0], v[1], v[2], v[3]};
                    else
                        for (int e = 0; e < 4 && n + e < g.N; ++e) dst[e] = v[e];
                } else {
                    uint16_t *dst = static_cast<uint16_t *>(g.c) + m * g.ldc + n;
                    const float sm = g.sa[m];
                    for (int e = 0; e < 4 && n + e < g.N; ++e) {
                        const float f = __fmul_rn(__fmul_rn(static_cast<float>(v[e]), sm), g.sb[n + e]);
                        dst[e] = round16<EPI == 2 ? NF4_BF16 : NF4_F16>(f);
                    }
                }
            }
    }
}

// Split-K finish: the int32 partials summed (exact, any order), written as int32 or scaled.
template <int EPI>
__global__ __launch_bounds__(256) void i8_reduce_kernel(const int32_t *partial, int splits,
                                                        int64_t M, int64_t N, const float *sa,
                                                        const float *sb, void *c, int64_t ldc) {
    const int64_t n = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t m = blockIdx.y;
    if (n >= N) return;
    int32_t acc = 0;
    for (int s = 0; s < splits; ++s) acc += partial[(static_cast<int64_t>(s) * M + m) * N + n];
    if constexpr (EPI == 0) {
        static_cast<int32_t *>(c)[m * ldc + n] = acc;
    } else {
        const float f = __fmul_rn(__fmul_rn(static_cast<float>(acc), sa[m]), sb[n]);
        static_cast<uint16_t *>(c)[m * ldc + n] = round16<EPI == 2 ? NF4_BF16 : NF4_F16>(f);
    }
}

// ------------------------------------------------------- SwiGLU backward, int8 requantized

// Row m (layer.py:414-442): dh = fp32(acc[m][j]) * sd[m] * cs[j]; with g, u the saved gate and
// up and sig = 1 / (1 + exp(-g)): d_gate = dh u sig (1 + g (1 - sig)), d_up = dh g sig;
// both halves requantized with one scale per row (largest |gradient| over the 2I values).
template <int DT>
__device__ __forceinline__ void swiglu_grads(int32_t acc, float sd, float cs, float g, float u,
                                             float &dg, float &du) {
    const float dh = __fmul_rn(__fmul_rn(static_cast<float>(acc), sd), cs);
    const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-g)));
    du = __fmul_rn(__fmul_rn(dh, g), sig);
    dg = __fmul_rn(__fmul_rn(__fmul_rn(dh, u), sig), __fadd_rn(1.0f, __fmul_rn(g, __fsub_rn(1.0f, sig))));
}

template <int DT>
__global__ __launch_bounds__(256) void int8_swiglu_bwd_kernel(const int32_t *acc, int64_t ldacc,
                                                              int64_t inter, const float *sd,
                                                              const float *cs, const uint16_t *gu,
                                                              int64_t ldgu, int8_t *q, int64_t ldq,
                                                              float *sq) {
    __shared__ float red[4];
    const int64_t m = blockIdx.x;
    const float sdm = sd[m];
    const int32_t *arow = acc + m * ldacc;
    const uint16_t *grow = gu + m * ldgu;
    float top = 0.0f;
    for (int64_t j = threadIdx.x; j < inter; j += 256) {
        float dg, du;
        swiglu_grads<DT>(arow[j], sdm, cs[j], load_act<DT>(grow + j), load_act<DT>(grow + inter + j), dg, du);
        top = fmaxf(top, fmaxf(fabsf(dg), fabsf(du)));
    }
    const float peak = fmaxf(block_max(top, red), 1e-20f);
    const float inv = __fdiv_rn(127.0f, peak);
    int8_t *qrow = q + m * ldq;
    for (int64_t j = threadIdx.x; j < inter; j += 256) {
        float dg, du;
        swiglu_grads<DT>(arow[j], sdm, cs[j], load_act<DT>(grow + j), load_act<DT>(grow + inter + j), dg, du);
        qrow[j] = static_cast<int8_t>(round_i8(__fmul_rn(dg, inv)));
        qrow[inter + j] = static_cast<int8_t>(round_i8(__fmul_rn(du, inv)));
    }
    if (threadIdx.x == 0) sq[m] = __fdiv_rn(peak, 127.0f);
}

// ------------------------------------------------------------------------------ host

int fill_stack(StackArgs &a, const nf4_weight *ws, int nw, int64_t tile_rows, bool need64) {
    if (!ws || nw < 1 || nw > kSegs) return NF4_ERR_ARG;
    a = StackArgs{};
    a.nseg = nw;
    a.cols = ws[0].cols;
    a.row0[0] = a.tile0[0] = 0;
    for (int i = 0; i < nw; ++i) {
        const int st = check_weight(&ws[i]);
        if (st != NF4_OK) return st;
        if (ws[i].cols != a.cols || ws[i].rows <= 0) return NF4_ERR_ARG;
        if (need64 && (ws[i].rows % 64 != 0 || ws[i].cols % 64 != 0 || ws[i].blocksize % 16 != 0 ||
                       !aligned(ws[i].packed, 8)))
            return NF4_ERR_UNSUPPORTED;
        a.w[i] = to_dev(ws[i]);
        a.row0[i + 1] = a.row0[i] + ws[i].rows;
        a.tile0[i + 1] = a.tile0[i] + (ws[i].rows + tile_rows - 1) / tile_rows;
    }
    if (a.cols <= 0 || a.cols % 2 != 0) return NF4_ERR_UNSUPPORTED;
    return NF4_OK;
}

int64_t colmax_tiles(const nf4_weight *ws, int nw) {
    int64_t t = 0;
    for (int i = 0; i < nw; ++i) t += (ws[i].rows + 255) / 256;
    return t;
}

}  // namespace

extern "C" size_t nf4_int8_colscale_workspace(const nf4_weight *ws, int nw) {
    if (!ws || nw < 1 || nw > kSegs) return 0;
    return static_cast<size_t>(colmax_tiles(ws, nw)) * ws[0].cols * sizeof(uint16_t);
}

extern "C" int nf4_int8_colscale(const nf4_weight *ws, int nw, float *scale, int dtype,
                                 void *workspace, size_t workspace_bytes, void *stream) {
    if (dtype != NF4_F16 && dtype != NF4_BF16) return NF4_ERR_ARG;
    StackArgs a;
    int st = fill_stack(a, ws, nw, 256, false);
    if (st != NF4_OK) return st;
    if (!scale) return NF4_ERR_ARG;
    const int64_t tiles = colmax_tiles(ws, nw);
    if (!workspace || workspace_bytes < nf4_int8_colscale_workspace(ws, nw)) return NF4_ERR_WORKSPACE;
    if (tiles > 65535) return NF4_ERR_UNSUPPORTED;
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint16_t *part = static_cast<uint16_t *>(workspace);
    const dim3 grid(static_cast<unsigned>((a.cols + 255) / 256), static_cast<unsigned>(tiles));
    const dim3 fgrid(static_cast<unsigned>((a.cols + 255) / 256));
    if (dtype == NF4_BF16) {
        hipLaunchKernelGGL(colmax_partial_kernel<NF4_BF16>, grid, dim3(256), 0, s, a, part);
        hipLaunchKernelGGL(colmax_final_kernel<NF4_BF16>, fgrid, dim3(256), 0, s, part, tiles, a.cols, scale);
    } else {
        hipLaunchKernelGGL(colmax_partial_kernel<NF4_F16>, grid, dim3(256), 0, s, a, part);
        hipLaunchKernelGGL(colmax_final_kernel<NF4_F16>, fgrid, dim3(256), 0, s, part, tiles, a.cols, scale);
    }
    return status_of(hipGetLastError());
}

extern "C" int nf4_int8_weight_t(const nf4_weight *ws, int nw, const float *scale, int8_t *q,
                                 int64_t ldq, void *stream) {
    StackArgs a;
    int st = fill_stack(a, ws, nw, 64, true);
    if (st != NF4_OK) return st;
    if (!scale || !q || ldq < a.row0[nw] || ldq % 16 != 0 || !aligned(q, 16)) return NF4_ERR_ARG;
    if (a.tile0[nw] > 65535) return NF4_ERR_UNSUPPORTED;
    const dim3 grid(static_cast<unsigned>(a.cols / 64), static_cast<unsigned>(a.tile0[nw]));
    hipLaunchKernelGGL(int8_weight_t_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       a, scale, q, ldq);
    return status_of(hipGetLastError());
}

extern "C" int nf4_int8_weight_rows(const nf4_weight *ws, int nw, int8_t *q, int64_t ldq, float *s,
                                    void *stream) {
    StackArgs a;
    int st = fill_stack(a, ws, nw, 64, false);
    if (st != NF4_OK) return st;
    if (!q || !s || ldq < a.cols) return NF4_ERR_ARG;
    const int64_t rows = a.row0[nw];
    if (rows > 0x7fffffff) return NF4_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(int8_weight_rows_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a, q, ldq, s);
    return status_of(hipGetLastError());
}

extern "C" int nf4_int8_rows(const void *x, int64_t rows, int64_t cols, int64_t ldx, int8_t *q,
                             int64_t ldq, float *s, int dtype, void *stream) {
    if (dtype != NF4_F16 && dtype != NF4_BF16 && dtype != NF4_F32) return NF4_ERR_ARG;
    if (rows < 0 || cols < 0 || (rows > 0 && (!x || !q || !s)) || ldx < cols || ldq < cols)
        return NF4_ERR_ARG;
    if (rows == 0 || cols == 0) return NF4_OK;
    if (cols % 8 != 0 || ldx % 8 != 0 || ldq % 8 != 0 || !aligned(x, 16) || !aligned(q, 8))
        return NF4_ERR_UNSUPPORTED;
    if (rows > 0x7fffffff) return NF4_ERR_UNSUPPORTED;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(rows));
    const uint8_t *xb = static_cast<const uint8_t *>(x);
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL(int8_rows_kernel<NF4_BF16>, grid, dim3(256), 0, st, xb, cols, ldx * 2, q, ldq, s);
    else if (dtype == NF4_F32)
        hipLaunchKernelGGL(int8_rows_kernel<NF4_F32>, grid, dim3(256), 0, st, xb, cols, ldx * 4, q, ldq, s);
    else
        hipLaunchKernelGGL(int8_rows_kernel<NF4_F16>, grid, dim3(256), 0, st, xb, cols, ldx * 2, q, ldq, s);
    return status_of(hipGetLastError());
}

namespace {

// Tile size and reduction splits: 256 x 256 tiles (one workgroup per CU) when they fill most of
// a round, else 128 x 128 (two per CU); splits fill the CUs' places, each keeping >= 8 steps.
struct I8Plan {
    int bt;
    int splits;
    int64_t m_tiles, tiles;
};

int i8_splits(int64_t tiles, int64_t steps, int64_t slots) {
    int s = 1;
    while (s < 16 && tiles * (s + 1) <= slots && steps / (s + 1) >= 8) ++s;
    while (s > 1 && (s - 1) * ((steps + s - 1) / s) >= steps) --s;
    return s;
}

// Cost: rounds x steps per workgroup x the measured step time (256 x 256: ~2.5 us with one
// workgroup per CU; 128 x 128: ~1.4 us with two per CU), plus ~10 us for a split's partials
// and reduction.
I8Plan i8_plan(int64_t m, int64_t n, int64_t k) {
    const int64_t steps = k / IBR;
    const int64_t mt2 = (m + 255) / 256, t2 = mt2 * ((n + 255) / 256);
    const int64_t mt1 = (m + 127) / 128, t1 = mt1 * ((n + 127) / 128);
    const int s2 = i8_splits(t2, steps, 256), s1 = i8_splits(t1, steps, 512);
    auto cost = [&](int64_t tiles, int s, int64_t slots, double t_step) {
        const int64_t rounds = (tiles * s + slots - 1) / slots;
        return double(rounds) * double((steps + s - 1) / s) * t_step + (s > 1 ? 10.0 : 0.0);
    };
    if (cost(t2, s2, 256, 2.5) < cost(t1, s1, 512, 1.4)) return I8Plan{256, s2, mt2, t2};
    return I8Plan{128, s1, mt1, t1};
}

}  // namespace

extern "C" size_t nf4_int8_gemm_workspace(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || k % IBR != 0) return 0;
    const I8Plan p = i8_plan(m, n, k);
    return p.splits > 1 ? static_cast<size_t>(p.splits) * m * n * sizeof(int32_t) : 0;
}

extern "C" int nf4_int8_gemm(const int8_t *a, int64_t m, int64_t lda, const int8_t *b, int64_t n,
                             int64_t ldb, int64_t k, const float *sa, const float *sb, void *c,
                             int64_t ldc, int out_dtype, void *workspace, size_t workspace_bytes,
                             void *stream) {
    if (out_dtype != NF4_I32 && out_dtype != NF4_F16 && out_dtype != NF4_BF16) return NF4_ERR_ARG;
    if (m < 0 || n < 0 || k < 0 || !c || ldc < n || lda < k || ldb < k) return NF4_ERR_ARG;
    if (m == 0 || n == 0) return NF4_OK;
    if (!a || !b || (out_dtype != NF4_I32 && (!sa || !sb))) return NF4_ERR_ARG;
    if (k % IBR != 0 || n % 4 != 0 || lda % 16 != 0 || ldb % 16 != 0 || !aligned(a, 16) ||
        !aligned(b, 16) || ldc % 4 != 0 || !aligned(c, 16))
        return NF4_ERR_UNSUPPORTED;
    // 32-bit in-window offsets: a 256-row window of either operand below 2 GiB
    if (256 * lda >= (int64_t(1) << 31) || 256 * ldb >= (int64_t(1) << 31)) return NF4_ERR_UNSUPPORTED;
    I8Args g{};
    g.a = a;
    g.b = b;
    g.M = m;
    g.N = n;
    g.K = k;
    g.lda = lda;
    g.ldb = ldb;
    g.sa = sa;
    g.sb = sb;
    g.c = c;
    g.ldc = ldc;
    const I8Plan p = i8_plan(m, n, k);
    g.m_tiles = p.m_tiles;
    const int64_t tiles = p.tiles;
    const int64_t steps = k / IBR;
    g.splits = p.splits;
    g.per_split = (steps + g.splits - 1) / g.splits;
    if (g.splits > 1) {
        if (!workspace || workspace_bytes < nf4_int8_gemm_workspace(m, n, k)) return NF4_ERR_WORKSPACE;
        g.partial = static_cast<int32_t *>(workspace);
    }
    if (tiles * g.splits > 0x7fffffff) return NF4_ERR_UNSUPPORTED;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(tiles * g.splits));
    if (p.bt == 256) {
        if (out_dtype == NF4_I32) hipLaunchKernelGGL((i8_gemm_kernel<0, 256>), grid, dim3(512), 0, st, g);
        else if (out_dtype == NF4_F16) hipLaunchKernelGGL((i8_gemm_kernel<1, 256>), grid, dim3(512), 0, st, g);
        else hipLaunchKernelGGL((i8_gemm_kernel<2, 256>), grid, dim3(512), 0, st, g);
    } else {
        if (out_dtype == NF4_I32) hipLaunchKernelGGL((i8_gemm_kernel<0, 128>), grid, dim3(256), 0, st, g);
        else if (out_dtype == NF4_F16) hipLaunchKernelGGL((i8_gemm_kernel<1, 128>), grid, dim3(256), 0, st, g);
        else hipLaunchKernelGGL((i8_gemm_kernel<2, 128>), grid, dim3(256), 0, st, g);
    }
    if (g.splits > 1) {
        if (m > 65535) return NF4_ERR_UNSUPPORTED;
        const dim3 rg(static_cast<unsigned>((n + 255) / 256), static_cast<unsigned>(m));
        if (out_dtype == NF4_I32)
            hipLaunchKernelGGL(i8_reduce_kernel<0>, rg, dim3(256), 0, st, g.partial, g.splits, m, n, sa, sb, c, ldc);
        else if (out_dtype == NF4_F16)
            hipLaunchKernelGGL(i8_reduce_kernel<1>, rg, dim3(256), 0, st, g.partial, g.splits, m, n, sa, sb, c, ldc);
        else
            hipLaunchKernelGGL(i8_reduce_kernel<2>, rg, dim3(256), 0, st, g.partial, g.splits, m, n, sa, sb, c, ldc);
    }
    return status_of(hipGetLastError());
}

extern "C" int nf4_int8_swiglu_bwd(const int32_t *acc, int64_t m, int64_t inter, int64_t ldacc,
                                   const float *sd, const float *cs, const void *gu, int64_t ldgu,
                                   int8_t *q, int64_t ldq, float *sq, int dtype, void *stream) {
    if (dtype != NF4_F16 && dtype != NF4_BF16) return NF4_ERR_ARG;
    if (m < 0 || inter < 0 || ldacc < inter || ldgu < 2 * inter || ldq < 2 * inter) return NF4_ERR_ARG;
    if (m == 0 || inter == 0) return NF4_OK;
    if (!acc || !sd || !cs || !gu || !q || !sq) return NF4_ERR_ARG;
    if (m > 0x7fffffff) return NF4_ERR_UNSUPPORTED;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(m));
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL(int8_swiglu_bwd_kernel<NF4_BF16>, grid, dim3(256), 0, st, acc, ldacc,
                           inter, sd, cs, static_cast<const uint16_t *>(gu), ldgu, q, ldq, sq);
    else
        hipLaunchKernelGGL(int8_swiglu_bwd_kernel<NF4_F16>, grid, dim3(256), 0, st, acc, ldacc,
                           inter, sd, cs, static_cast<const uint16_t *>(gu), ldgu, q, ldq, sq);
    return status_of(hipGetLastError());
}
