// Fused NF4 dequant-GEMMs for gfx950 (MI355X): forward Y = X W^T and input gradient
// dX = dY W, with W dequantized inside the main loop and the LoRA terms folded in as extra
// rank-16 reduction slabs.
//
// Reference arithmetic replaced: F.linear / addmm / mm on the fp16 weight that
// nf4_dequant_kernel wrote (/root/reference/solution/nf4.py:84-102; layer.py:871-878, 893,
// 914, 929, 1015-1033, 1061, 1072-1090; mlp.py:42-74).
//
// Both GEMMs are computed transposed, C[p, m] = sum_r Wop[p, r] * Act[m, r], so that the MFMA
// "A" operand is the weight side (rows p) and the "B" operand the activation rows m:
//   forward: p = n (output feature), r = k, Wop = W          (natural layout)
//   dX:      p = k (input feature),  r = n, Wop = W^T        (transposed while dequantizing)
// With v_mfma_f32_32x32x16 each lane then owns one activation row m and four consecutive p,
// so results leave as 8-byte row-major stores of Y[m, n..n+3] or dX[m, k..k+3].
//
// Workgroup tile BP x BM, reduction step 64 (one NF4 absmax block along k for the forward
// weight), two LDS stages.  LDS tiles are rows of 64 16-bit values (128 bytes) whose 16-byte
// chunks are XOR-swizzled by the row index, so MFMA fragment reads of 32 consecutive rows spread
// over the banks.  Per step:
//   * the activation tile of the next step streams straight from global memory into the other
//     LDS stage (global_load_lds_dwordx4, no registers; lanes pick their global chunk so that
//     the lane-linear LDS writes land in the swizzled layout);
//   * the packed weight bytes of the next step (4x smaller than fp16) are prefetched into
//     registers;
//   * the MFMAs of the current step run; meanwhile the other wave on the same SIMD dequantizes
//     (NF4 table in LDS, absmax rebuilt from its uint8 code, fp32 product, one RNE conversion)
//     and writes the next weight tile to LDS;
//   * one barrier.
// Long reductions are split over workgroups into fp32 partial sums that a reduction kernel
// adds up in a fixed order (deterministic).

#include "nf4_common.h"

namespace {

constexpr int BR = 64;           // reduction step
constexpr int ROWB = 128;        // bytes per LDS tile row
constexpr int kMaxSeg = NF4_MAX_SEGMENTS;

typedef __attribute__((address_space(3))) void lds_void;

// Byte offset of 16-byte chunk c (elements 8c..8c+7) of row r in an LDS tile.
__device__ __forceinline__ int swz(int r, int c) { return r * ROWB + ((c ^ (r & 7)) << 4); }

struct LoraDev {
    const uint16_t *t;   // forward: [M, rank]
    const uint16_t *b;   // forward: [rows_seg, rank]
    const uint16_t *a;   // dx: [rank, K]
    const uint16_t *da;  // dx: [M, rank]
    float scale;
    int rank;
    int has;
};

struct GemmArgs {
    const uint16_t *act;          // X (forward) or dY (dx)
    int64_t ld_act;
    int64_t M;
    int64_t K;                    // in_features of every segment
    DevWeight w[kMaxSeg];
    int64_t seg_off[kMaxSeg];     // forward: output column offset; dx: dY column offset
    int64_t tile_start[kMaxSeg + 1];  // forward: cumulative (p tiles x m tiles) per segment
    int64_t step_start[kMaxSeg + 1];  // dx: cumulative reduction steps per segment
    int nseg;
    LoraDev lora[kMaxSeg];
    const uint16_t *bias;         // forward: [sum rows] or null
    void *out;
    int64_t ld_out;
    int64_t n_out;                // forward: sum rows; dx: K
    float *partial;               // split workspace [splits][M][n_out] or null
    int splits;
    int64_t m_tiles;
    int64_t p_tiles;              // dx: tiles along K
    int64_t total_steps;          // dx: sum of step counts
    int accumulate;               // dx: add into out
    int vec_out;                  // 8-byte output stores allowed
};

template <int DT>
__device__ __forceinline__ float16_t mfma32(const u32x4_t &a, const u32x4_t &b, const float16_t &c) {
    if constexpr (DT == NF4_BF16) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf168_t, a),
                                                      __builtin_bit_cast(bf168_t, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a),
                                                     __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
    }
}

template <int DT>
__device__ __forceinline__ float to_f32(uint16_t v) {
    if constexpr (DT == NF4_BF16) return __uint_as_float(static_cast<uint32_t>(v) << 16);
    else return static_cast<float>(__builtin_bit_cast(half_t, v));
}

template <int DT>
__device__ __forceinline__ uint16_t from_f32(float v) {
    if constexpr (DT == NF4_BF16) return __builtin_bit_cast(uint16_t, static_cast<bf16_t>(v));
    else return __builtin_bit_cast(uint16_t, static_cast<half_t>(v));
}

// 8 NF4 codes of one dword (byte j: high nibble = element 2j, low = 2j+1) times absmax,
// rounded once to DT and packed.
template <int DT>
__device__ __forceinline__ u32x4_t dequant8(uint32_t p, float s, const float *code) {
    u32x4_t r;
    r.x = pack2<DT>(__fmul_rn(code[(p >> 4) & 0xF], s), __fmul_rn(code[p & 0xF], s));
    r.y = pack2<DT>(__fmul_rn(code[(p >> 12) & 0xF], s), __fmul_rn(code[(p >> 8) & 0xF], s));
    r.z = pack2<DT>(__fmul_rn(code[(p >> 20) & 0xF], s), __fmul_rn(code[(p >> 16) & 0xF], s));
    r.w = pack2<DT>(__fmul_rn(code[(p >> 28) & 0xF], s), __fmul_rn(code[(p >> 24) & 0xF], s));
    return r;
}

__device__ __forceinline__ int seg_of_tile(const GemmArgs &a, int64_t t) {
    int s = 0;
#pragma unroll
    for (int i = 1; i < kMaxSeg; ++i)
        if (i < a.nseg && t >= a.tile_start[i]) s = i;
    return s;
}

__device__ __forceinline__ int seg_of_step(const GemmArgs &a, int64_t t) {
    int s = 0;
#pragma unroll
    for (int i = 1; i < kMaxSeg; ++i)
        if (i < a.nseg && t >= a.step_start[i]) s = i;
    return s;
}

// The raw absmax inputs of block b, fetched with the packed bytes; rebuilt later by absmax_val.
struct AbsIn {
    float s;      // absmax2 scale (nested) or the fp32 absmax
    uint32_t q;   // uint8 code (nested)
};

__device__ __forceinline__ AbsIn absmax_load(const DevWeight &w, int64_t b) {
    AbsIn r;
    if (w.nested) {
        r.q = static_cast<const uint8_t *>(w.absmax)[b];
        r.s = w.absmax2[b / w.blocksize2];
    } else {
        r.q = 0;
        r.s = static_cast<const float *>(w.absmax)[b];
    }
    return r;
}

__device__ __forceinline__ float absmax_val(const DevWeight &w, const AbsIn &in, const float *code2) {
    return w.nested ? __fadd_rn(__fmul_rn(code2[in.q], in.s), w.offset) : in.s;
}

// ------------------------------------------------------------------ activation tile loader

// BM rows x 64 columns of act[m][col0 ..] into an LDS tile.  Full-width steps stream straight
// into LDS; rows past M re-read row M-1 (their results are never stored).
template <int BM, int NT>
__device__ __forceinline__ void act_load_direct(const GemmArgs &a, uint8_t *s, int64_t m0,
                                                int64_t col0) {
    constexpr int REGIONS = BM * ROWB / 1024;   // 1 KB = 8 rows per wave instruction
    constexpr int WAVES = NT / 64;
    static_assert(REGIONS % WAVES == 0, "tile rows must split evenly over the waves");
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < REGIONS / WAVES; ++i) {
        const int region = i * WAVES + wave;
        const int r = region * 8 + (lane >> 3);
        const int c = (lane & 7) ^ (r & 7);      // this lane's slot holds logical chunk c
        int64_t m = m0 + r;
        m = m < a.M ? m : a.M - 1;
        __builtin_amdgcn_global_load_lds(a.act + m * a.ld_act + col0 + c * 8,
                                         (lds_void *)(s + region * 1024), 16, 0, 0);
    }
}

// Same tile with columns >= col_end read as zero (a segment's last, partial reduction step).
template <int BM, int NT>
__device__ __forceinline__ void act_load_masked(const GemmArgs &a, uint8_t *s, int64_t m0,
                                                int64_t col0, int64_t col_end) {
    for (int idx = threadIdx.x; idx < BM * 8; idx += NT) {
        const int r = idx >> 3, c = idx & 7;
        const int64_t m = m0 + r;
        const int64_t cc = col0 + c * 8;
        uint16_t e[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (m < a.M) {
            const uint16_t *src = a.act + m * a.ld_act + cc;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (cc + j < col_end) e[j] = src[j];
        }
        u32x4_t v;
        v.x = e[0] | (uint32_t(e[1]) << 16);
        v.y = e[2] | (uint32_t(e[3]) << 16);
        v.z = e[4] | (uint32_t(e[5]) << 16);
        v.w = e[6] | (uint32_t(e[7]) << 16);
        *reinterpret_cast<u32x4_t *>(s + swz(r, c)) = v;
    }
}

// ------------------------------------------------------------------------- MFMA core

// Wave-level MFMA over one 64-deep step: acc[TP][TM] += Wop[p rows] x Act[m rows].
template <int DT, int TP, int TM>
__device__ __forceinline__ void mma_step(float16_t (&acc)[TP][TM], const uint8_t *sw,
                                         const uint8_t *sa, int prow0, int mrow0) {
    const int lane = threadIdx.x & 63;
    const int r = lane & 31;
    const int kh = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < BR / 16; ++ks) {
        const int c = ks * 2 + kh;
        u32x4_t fa[TP], fb[TM];
#pragma unroll
        for (int i = 0; i < TP; ++i)
            fa[i] = *reinterpret_cast<const u32x4_t *>(sw + swz(prow0 + i * 32 + r, c));
#pragma unroll
        for (int j = 0; j < TM; ++j)
            fb[j] = *reinterpret_cast<const u32x4_t *>(sa + swz(mrow0 + j * 32 + r, c));
#pragma unroll
        for (int i = 0; i < TP; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) acc[i][j] = mfma32<DT>(fa[i], fb[j], acc[i][j]);
    }
}

// 8 16-bit values at src[j * stride] (j < lim) packed into an MFMA fragment.
__device__ __forceinline__ u32x4_t gather8(const uint16_t *src, int64_t stride, int lim) {
    uint16_t e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = (j < lim) ? src[j * stride] : 0;
    u32x4_t v;
    v.x = e[0] | (uint32_t(e[1]) << 16);
    v.y = e[2] | (uint32_t(e[3]) << 16);
    v.z = e[4] | (uint32_t(e[5]) << 16);
    v.w = e[6] | (uint32_t(e[7]) << 16);
    return v;
}

// Epilogue: lane holds C[p .. p+3][m] for each (i, j, r4).  Writes either fp32 partials
// (split mode) or final values (+bias, +existing for accumulate) in DT.
template <int DT, int TP, int TM>
__device__ __forceinline__ void epilogue(const GemmArgs &a, float16_t (&acc)[TP][TM],
                                         int64_t p_base, int64_t p_end, int64_t col_off,
                                         int64_t m_base, int split) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const int64_t m = m_base + j * 32 + (lane & 31);
        if (m >= a.M) continue;
#pragma unroll
        for (int i = 0; i < TP; ++i) {
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int64_t p = p_base + i * 32 + r4 * 8 + (lane >> 5) * 4;
                if (p >= p_end) continue;
                const int64_t col = col_off + p;
                float v[4] = {acc[i][j][r4 * 4 + 0], acc[i][j][r4 * 4 + 1],
                              acc[i][j][r4 * 4 + 2], acc[i][j][r4 * 4 + 3]};
                const bool full = p + 4 <= p_end;
                if (a.partial) {
                    float *dst = a.partial + (static_cast<int64_t>(split) * a.M + m) * a.n_out + col;
                    if (full) {
                        *reinterpret_cast<float4_t *>(dst) = (float4_t){v[0], v[1], v[2], v[3]};
                    } else {
                        for (int q = 0; q < 4; ++q)
                            if (p + q < p_end) dst[q] = v[q];
                    }
                    continue;
                }
                uint16_t *dst = static_cast<uint16_t *>(a.out) + m * a.ld_out + col;
                if (a.bias) {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (p + q < p_end) v[q] += to_f32<DT>(a.bias[col + q]);
                }
                if (full && a.vec_out) {
                    if (a.accumulate) {
                        const u32x2_t old = *reinterpret_cast<const u32x2_t *>(dst);
                        v[0] += to_f32<DT>(old.x & 0xffff);
                        v[1] += to_f32<DT>(old.x >> 16);
                        v[2] += to_f32<DT>(old.y & 0xffff);
                        v[3] += to_f32<DT>(old.y >> 16);
                    }
                    u32x2_t o;
                    o.x = pack2<DT>(v[0], v[1]);
                    o.y = pack2<DT>(v[2], v[3]);
                    *reinterpret_cast<u32x2_t *>(dst) = o;
                } else {
                    for (int q = 0; q < 4; ++q) {
                        if (p + q >= p_end) break;
                        float x = v[q];
                        if (a.accumulate) x += to_f32<DT>(dst[q]);
                        dst[q] = from_f32<DT>(x);
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------------ weight tiles

// Forward weight tile: BP rows x 64 k of W (natural layout).  Thread t owns 16 packed bytes =
// 32 elements of row t/2 (one absmax); NT == 2 * BP.
template <int DT, int BP>
struct FwdWeight {
    u32x4_t raw;
    AbsIn abs;

    __device__ __forceinline__ void load(const DevWeight &w, int64_t p0, int64_t K, int64_t st) {
        const int row = threadIdx.x >> 1;
        const int64_t n = p0 + row;
        raw = (u32x4_t){0u, 0u, 0u, 0u};
        abs = AbsIn{0.f, 0u};
        if (n < w.rows) {
            const int64_t e0 = n * K + st * BR;
            raw = *reinterpret_cast<const u32x4_t *>(w.packed + (e0 >> 1) + (threadIdx.x & 1) * 16);
            abs = absmax_load(w, e0 / w.blocksize);
        }
    }

    __device__ __forceinline__ void store(const DevWeight &w, uint8_t *s, const float *code,
                                          const float *code2) const {
        const int row = threadIdx.x >> 1, h = (threadIdx.x & 1) * 4;
        const float sc = absmax_val(w, abs, code2);
        *reinterpret_cast<u32x4_t *>(s + swz(row, h + 0)) = dequant8<DT>(raw.x, sc, code);
        *reinterpret_cast<u32x4_t *>(s + swz(row, h + 1)) = dequant8<DT>(raw.y, sc, code);
        *reinterpret_cast<u32x4_t *>(s + swz(row, h + 2)) = dequant8<DT>(raw.z, sc, code);
        *reinterpret_cast<u32x4_t *>(s + swz(row, h + 3)) = dequant8<DT>(raw.w, sc, code);
    }
};

// dX weight tile: 64 n x BP k of W, written transposed (LDS rows = k).  Thread t owns a patch
// of 4 rows n x 8 columns k (one dword per row, one absmax per row); NT == 2 * BP.
template <int DT, int BP>
struct DxWeight {
    static constexpr int KG = BP / 8;
    uint32_t raw[4];
    AbsIn abs[4];

    __device__ __forceinline__ void load(const DevWeight &w, int64_t n0, int64_t p0, int64_t K) {
        const int kg = threadIdx.x % KG, ng = threadIdx.x / KG;
        const int64_t k = p0 + kg * 8;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t n = n0 + ng * 4 + i;
            raw[i] = 0u;
            abs[i] = AbsIn{0.f, 0u};
            if (n < w.rows && k < K) {
                const int64_t e0 = n * K + k;
                raw[i] = *reinterpret_cast<const uint32_t *>(w.packed + (e0 >> 1));
                abs[i] = absmax_load(w, e0 / w.blocksize);
            }
        }
    }

    __device__ __forceinline__ void store(const DevWeight &w, uint8_t *s, const float *code,
                                          const float *code2) const {
        const int kg = threadIdx.x % KG, ng = threadIdx.x / KG;
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = absmax_val(w, abs[i], code2);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int sh = (e & 1) ? (e >> 1) * 8 : (e >> 1) * 8 + 4;
            u32x2_t o;
            o.x = pack2<DT>(__fmul_rn(code[(raw[0] >> sh) & 0xF], sc[0]),
                            __fmul_rn(code[(raw[1] >> sh) & 0xF], sc[1]));
            o.y = pack2<DT>(__fmul_rn(code[(raw[2] >> sh) & 0xF], sc[2]),
                            __fmul_rn(code[(raw[3] >> sh) & 0xF], sc[3]));
            *reinterpret_cast<u32x2_t *>(s + swz(kg * 8 + e, ng >> 1) + (ng & 1) * 8) = o;
        }
    }
};

// ------------------------------------------------------------------------------- kernels

template <int DT, int BP, int BM, int WP, int WM>
__global__ __launch_bounds__(WP *WM * 64) void fwd_kernel(const GemmArgs a) {
    constexpr int NT = WP * WM * 64;
    constexpr int TP = BP / WP / 32, TM = BM / WM / 32;
    static_assert(NT == 2 * BP, "forward weight tile mapping needs 2 threads per row");
    __shared__ __attribute__((aligned(1024))) uint8_t sW[2][BP * ROWB];
    __shared__ __attribute__((aligned(1024))) uint8_t sA[2][BM * ROWB];
    __shared__ float s_code[16];
    __shared__ float s_code2[256];

    const int64_t bid = blockIdx.x;
    const int split = static_cast<int>(bid % a.splits);
    const int64_t tile = bid / a.splits;
    const int seg = seg_of_tile(a, tile);
    const int64_t local = tile - a.tile_start[seg];
    const int64_t p0 = (local / a.m_tiles) * BP;
    const int64_t m0 = (local % a.m_tiles) * BM;
    const DevWeight &w = a.w[seg];
    const int64_t K = a.K;
    const int64_t steps = K / BR;
    const int64_t per = (steps + a.splits - 1) / a.splits;
    const int64_t s0 = split * per;
    const int64_t s1 = s0 + per < steps ? s0 + per : steps;

    for (int i = threadIdx.x; i < 16; i += NT) s_code[i] = w.code[i];
    if (w.nested)
        for (int i = threadIdx.x; i < 256; i += NT) s_code2[i] = w.code2[i];

    const int wave = threadIdx.x >> 6;
    const int wp = wave % WP, wm = wave / WP;
    const int lane = threadIdx.x & 63;

    float16_t acc[TP][TM];
#pragma unroll
    for (int i = 0; i < TP; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = (float16_t){};

    // LoRA slab(s): acc = scale * B[p rows] . T[m rows]^T, before the weight product.
    const LoraDev &lo = a.lora[seg];
    if (lo.has && split == 0) {
        const int r = lane & 31, kh = (lane >> 5) * 8;
        for (int k0 = 0; k0 < lo.rank; k0 += 16) {
            const int lim = lo.rank - (k0 + kh);
            u32x4_t fa[TP], fb[TM];
#pragma unroll
            for (int i = 0; i < TP; ++i) {
                const int64_t p = p0 + wp * (BP / WP) + i * 32 + r;
                fa[i] = (p < w.rows && lim > 0) ? gather8(lo.b + p * lo.rank + k0 + kh, 1, lim)
                                                : (u32x4_t){0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int64_t m = m0 + wm * (BM / WM) + j * 32 + r;
                fb[j] = (m < a.M && lim > 0) ? gather8(lo.t + m * lo.rank + k0 + kh, 1, lim)
                                             : (u32x4_t){0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int i = 0; i < TP; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j) acc[i][j] = mfma32<DT>(fa[i], fb[j], acc[i][j]);
        }
#pragma unroll
        for (int i = 0; i < TP; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) acc[i][j] *= lo.scale;
    }

    FwdWeight<DT, BP> wt;
    __syncthreads();  // tables
    if (s0 < s1) {
        act_load_direct<BM, NT>(a, sA[0], m0, s0 * BR);
        wt.load(w, p0, K, s0);
        wt.store(w, sW[0], s_code, s_code2);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        for (int64_t st = s0; st < s1; ++st) {
            const int buf = static_cast<int>((st - s0) & 1);
            const bool more = st + 1 < s1;
            if (more) {
                act_load_direct<BM, NT>(a, sA[buf ^ 1], m0, (st + 1) * BR);
                wt.load(w, p0, K, st + 1);
            }
            mma_step<DT, TP, TM>(acc, sW[buf], sA[buf], wp * (BP / WP), wm * (BM / WM));
            if (more) wt.store(w, sW[buf ^ 1], s_code, s_code2);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
    }
    epilogue<DT, TP, TM>(a, acc, p0 + wp * (BP / WP), w.rows, a.seg_off[seg],
                         m0 + wm * (BM / WM), split);
}

template <int DT, int BP, int BM, int WP, int WM>
__global__ __launch_bounds__(WP *WM * 64) void dx_kernel(const GemmArgs a) {
    constexpr int NT = WP * WM * 64;
    constexpr int TP = BP / WP / 32, TM = BM / WM / 32;
    static_assert(NT == 2 * BP, "dX weight tile mapping needs 2 threads per k column group");
    __shared__ __attribute__((aligned(1024))) uint8_t sW[2][BP * ROWB];
    __shared__ __attribute__((aligned(1024))) uint8_t sA[2][BM * ROWB];
    __shared__ float s_code[kMaxSeg][16];
    __shared__ float s_code2[kMaxSeg][256];

    const int64_t bid = blockIdx.x;
    const int split = static_cast<int>(bid % a.splits);
    const int64_t tile = bid / a.splits;
    const int64_t p0 = (tile / a.m_tiles) * BP;
    const int64_t m0 = (tile % a.m_tiles) * BM;
    const int64_t K = a.K;
    const int64_t per = (a.total_steps + a.splits - 1) / a.splits;
    const int64_t s0 = split * per;
    const int64_t s1 = s0 + per < a.total_steps ? s0 + per : a.total_steps;

    for (int s = 0; s < a.nseg; ++s) {
        for (int i = threadIdx.x; i < 16; i += NT) s_code[s][i] = a.w[s].code[i];
        if (a.w[s].nested)
            for (int i = threadIdx.x; i < 256; i += NT) s_code2[s][i] = a.w[s].code2[i];
    }

    const int wave = threadIdx.x >> 6;
    const int wp = wave % WP, wm = wave / WP;
    const int lane = threadIdx.x & 63;

    float16_t acc[TP][TM];
#pragma unroll
    for (int i = 0; i < TP; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = (float16_t){};

    // LoRA slabs: acc += A^T[k rows] . da[m rows]^T (reduction over the rank).
    if (split == 0) {
        const int r = lane & 31, kh = (lane >> 5) * 8;
        for (int s = 0; s < a.nseg; ++s) {
            const LoraDev &lo = a.lora[s];
            if (!lo.has) continue;
            for (int k0 = 0; k0 < lo.rank; k0 += 16) {
                const int lim = lo.rank - (k0 + kh);
                u32x4_t fa[TP], fb[TM];
#pragma unroll
                for (int i = 0; i < TP; ++i) {
                    const int64_t p = p0 + wp * (BP / WP) + i * 32 + r;
                    fa[i] = (p < K && lim > 0) ? gather8(lo.a + (k0 + kh) * K + p, K, lim)
                                               : (u32x4_t){0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int j = 0; j < TM; ++j) {
                    const int64_t m = m0 + wm * (BM / WM) + j * 32 + r;
                    fb[j] = (m < a.M && lim > 0) ? gather8(lo.da + m * lo.rank + k0 + kh, 1, lim)
                                                 : (u32x4_t){0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int i = 0; i < TP; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j) acc[i][j] = mfma32<DT>(fa[i], fb[j], acc[i][j]);
            }
        }
    }

    DxWeight<DT, BP> wt;
    // One reduction step: segment seg, rows n0 .. n0+64 of it.
    auto load_step = [&](int64_t st, uint8_t *sa_buf, int &seg) {
        seg = seg_of_step(a, st);
        const int64_t n0 = (st - a.step_start[seg]) * BR;
        const int64_t rows = a.w[seg].rows;
        const int64_t col0 = a.seg_off[seg] + n0;
        if (n0 + BR <= rows) act_load_direct<BM, NT>(a, sa_buf, m0, col0);
        else act_load_masked<BM, NT>(a, sa_buf, m0, col0, a.seg_off[seg] + rows);
        wt.load(a.w[seg], n0, p0, K);
    };

    __syncthreads();  // tables
    if (s0 < s1) {
        int seg;
        load_step(s0, sA[0], seg);
        wt.store(a.w[seg], sW[0], s_code[seg], s_code2[seg]);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        for (int64_t st = s0; st < s1; ++st) {
            const int buf = static_cast<int>((st - s0) & 1);
            const bool more = st + 1 < s1;
            if (more) load_step(st + 1, sA[buf ^ 1], seg);
            mma_step<DT, TP, TM>(acc, sW[buf], sA[buf], wp * (BP / WP), wm * (BM / WM));
            if (more) wt.store(a.w[seg], sW[buf ^ 1], s_code[seg], s_code2[seg]);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
    }
    epilogue<DT, TP, TM>(a, acc, p0 + wp * (BP / WP), K, 0, m0 + wm * (BM / WM), split);
}

// Split reduction: out[m][c] = sum_s partial[s][m][c] (+bias[c]) (+out if accumulate).
template <int DT>
__global__ __launch_bounds__(256) void split_reduce_kernel(const float *partial, int splits,
                                                           int64_t M, int64_t n_out,
                                                           const uint16_t *bias, uint16_t *out,
                                                           int64_t ld_out, int accumulate) {
    const int64_t total = M * n_out;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t m = i / n_out, c = i % n_out;
        float v = 0.f;
        for (int s = 0; s < splits; ++s) v += partial[s * total + i];
        if (bias) v += to_f32<DT>(bias[c]);
        uint16_t *dst = out + m * ld_out + c;
        if (accumulate) v += to_f32<DT>(*dst);
        *dst = from_f32<DT>(v);
    }
}

// ------------------------------------------------------------------------------ host side

struct Plan {
    int cfg;       // 0: 256x256 tile / 8 waves, 1: 128x128 tile / 4 waves
    int bp, bm;
    int splits;
    int64_t tiles;
};

constexpr int kCUs = 256;

int fill_common(GemmArgs &g, const void *act, int64_t m, int64_t ld_act, const nf4_weight *ws,
                int nw) {
    if (!ws || nw < 1 || nw > kMaxSeg) return NF4_ERR_ARG;
    g = GemmArgs{};
    g.act = static_cast<const uint16_t *>(act);
    g.ld_act = ld_act;
    g.M = m;
    g.nseg = nw;
    g.K = ws[0].cols;
    for (int i = 0; i < nw; ++i) {
        const int st = check_weight(&ws[i]);
        if (st != NF4_OK) return st;
        if (ws[i].cols != g.K) return NF4_ERR_ARG;
        // The fused main loop needs each 64-wide step of a weight row inside one absmax block.
        if (ws[i].blocksize % BR != 0 || g.K % ws[i].blocksize != 0) return NF4_ERR_UNSUPPORTED;
        if (!aligned(ws[i].packed, 16)) return NF4_ERR_UNSUPPORTED;
        g.w[i] = to_dev(ws[i]);
    }
    if (g.K % BR != 0 || ld_act % 8 != 0 || !aligned(act, 16)) return NF4_ERR_UNSUPPORTED;
    return NF4_OK;
}

// Splits of the reduction so that about one round of workgroups covers the GPU, keeping at
// least 8 steps per split.
int choose_splits(int64_t tiles, int64_t steps, int per_cu) {
    int s = 1;
    while (tiles * s * 2 <= kCUs * per_cu && steps / (s * 2) >= 8 && s < 16) s *= 2;
    return s;
}

Plan make_plan(int64_t big, int64_t small, int64_t steps) {
    Plan p{};
    if (big >= kCUs) {
        p.cfg = 0; p.bp = 256; p.bm = 256; p.tiles = big;
        p.splits = choose_splits(big, steps, 1);
    } else {
        p.cfg = 1; p.bp = 128; p.bm = 128; p.tiles = small;
        p.splits = choose_splits(small, steps, 2);
    }
    return p;
}

Plan plan_fwd(int64_t m, const nf4_weight *ws, int nw) {
    int64_t big = 0, small = 0;
    for (int i = 0; i < nw; ++i) {
        big += (ws[i].rows + 255) / 256;
        small += (ws[i].rows + 127) / 128;
    }
    big *= (m + 255) / 256;
    small *= (m + 127) / 128;
    return make_plan(big, small, ws[0].cols / BR);
}

Plan plan_dx(int64_t m, const nf4_weight *ws, int nw) {
    int64_t steps = 0;
    for (int i = 0; i < nw; ++i) steps += (ws[i].rows + BR - 1) / BR;
    const int64_t K = ws[0].cols;
    const int64_t big = ((K + 255) / 256) * ((m + 255) / 256);
    const int64_t small = ((K + 127) / 128) * ((m + 127) / 128);
    return make_plan(big, small, steps);
}

template <int DT>
int launch_fwd(const GemmArgs &g, const Plan &p, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(p.tiles * p.splits));
    if (p.cfg == 0)
        hipLaunchKernelGGL((fwd_kernel<DT, 256, 256, 2, 4>), grid, dim3(512), 0, st, g);
    else
        hipLaunchKernelGGL((fwd_kernel<DT, 128, 128, 2, 2>), grid, dim3(256), 0, st, g);
    return status_of(hipGetLastError());
}

template <int DT>
int launch_dx(const GemmArgs &g, const Plan &p, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(p.tiles * p.splits));
    if (p.cfg == 0)
        hipLaunchKernelGGL((dx_kernel<DT, 256, 256, 2, 4>), grid, dim3(512), 0, st, g);
    else
        hipLaunchKernelGGL((dx_kernel<DT, 128, 128, 2, 2>), grid, dim3(256), 0, st, g);
    return status_of(hipGetLastError());
}

template <int DT>
int launch_reduce(const GemmArgs &g, int splits, hipStream_t st) {
    const int64_t total = g.M * g.n_out;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(split_reduce_kernel<DT>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       st, g.partial, splits, g.M, g.n_out, g.bias,
                       static_cast<uint16_t *>(g.out), g.ld_out, g.accumulate);
    return status_of(hipGetLastError());
}

}  // namespace

extern "C" size_t nf4_linear_fwd_workspace(int64_t m, const nf4_weight *ws, int nw, int dtype) {
    (void)dtype;
    if (!ws || nw < 1 || nw > kMaxSeg || m <= 0) return 0;
    const Plan p = plan_fwd(m, ws, nw);
    if (p.splits <= 1) return 0;
    int64_t n = 0;
    for (int i = 0; i < nw; ++i) n += ws[i].rows;
    return static_cast<size_t>(p.splits) * m * n * sizeof(float);
}

extern "C" size_t nf4_linear_dx_workspace(int64_t m, const nf4_weight *ws, int nw, int dtype) {
    (void)dtype;
    if (!ws || nw < 1 || nw > kMaxSeg || m <= 0) return 0;
    const Plan p = plan_dx(m, ws, nw);
    if (p.splits <= 1) return 0;
    return static_cast<size_t>(p.splits) * m * ws[0].cols * sizeof(float);
}

extern "C" int nf4_linear_fwd(const void *x, int64_t m, int64_t ldx, const nf4_weight *ws, int nw,
                              const void *bias, const nf4_lora *loras, int nlora, void *y,
                              int64_t ldy, int dtype, void *workspace, size_t workspace_bytes,
                              void *stream) {
    if (dtype != NF4_F16 && dtype != NF4_BF16) return NF4_ERR_ARG;
    if (m < 0 || !y || (m > 0 && !x) || nlora < 0 || (nlora > 0 && !loras)) return NF4_ERR_ARG;
    GemmArgs g;
    int st = fill_common(g, x, m, ldx, ws, nw);
    if (st != NF4_OK) return st;
    int64_t n_out = 0;
    for (int i = 0; i < nw; ++i) {
        g.seg_off[i] = n_out;
        n_out += ws[i].rows;
    }
    if (ldy < n_out) return NF4_ERR_ARG;
    for (int i = 0; i < nlora; ++i) {
        const nf4_lora &l = loras[i];
        if (l.seg < 0 || l.seg >= nw || l.rank < 1 || l.rank > 64 || !l.t || !l.b) return NF4_ERR_ARG;
        LoraDev &d = g.lora[l.seg];
        if (d.has) return NF4_ERR_ARG;
        d.t = static_cast<const uint16_t *>(l.t);
        d.b = static_cast<const uint16_t *>(l.b);
        d.rank = l.rank;
        d.scale = l.scale;
        d.has = 1;
    }
    if (m == 0 || n_out == 0) return NF4_OK;
    g.bias = static_cast<const uint16_t *>(bias);
    g.out = y;
    g.ld_out = ldy;
    g.n_out = n_out;
    g.vec_out = aligned(y, 8) && ldy % 4 == 0;
    for (int i = 0; i < nw; ++i) g.vec_out = g.vec_out && (g.seg_off[i] % 4 == 0);
    const Plan p = plan_fwd(m, ws, nw);
    g.splits = p.splits;
    const int64_t bp = p.bp, bm = p.bm;
    g.m_tiles = (m + bm - 1) / bm;
    g.tile_start[0] = 0;
    for (int i = 0; i < nw; ++i)
        g.tile_start[i + 1] = g.tile_start[i] + ((ws[i].rows + bp - 1) / bp) * g.m_tiles;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (p.splits > 1) {
        const size_t need = static_cast<size_t>(p.splits) * m * n_out * sizeof(float);
        if (!workspace || workspace_bytes < need) return NF4_ERR_WORKSPACE;
        g.partial = static_cast<float *>(workspace);
    }
    st = dtype == NF4_BF16 ? launch_fwd<NF4_BF16>(g, p, s) : launch_fwd<NF4_F16>(g, p, s);
    if (st != NF4_OK || p.splits <= 1) return st;
    return dtype == NF4_BF16 ? launch_reduce<NF4_BF16>(g, p.splits, s)
                             : launch_reduce<NF4_F16>(g, p.splits, s);
}

extern "C" int nf4_linear_dx(const void *dy, int64_t m, int64_t lddy, const nf4_weight *ws, int nw,
                             const nf4_lora *loras, int nlora, void *dx, int64_t lddx,
                             int accumulate, int dtype, void *workspace, size_t workspace_bytes,
                             void *stream) {
    if (dtype != NF4_F16 && dtype != NF4_BF16) return NF4_ERR_ARG;
    if (m < 0 || !dx || (m > 0 && !dy) || nlora < 0 || (nlora > 0 && !loras)) return NF4_ERR_ARG;
    GemmArgs g;
    int st = fill_common(g, dy, m, lddy, ws, nw);
    if (st != NF4_OK) return st;
    int64_t n_in = 0;
    for (int i = 0; i < nw; ++i) {
        g.seg_off[i] = n_in;
        if (n_in % 8 != 0) return NF4_ERR_UNSUPPORTED;  // 16-byte dY loads per segment
        n_in += ws[i].rows;
    }
    if (lddy < n_in || lddx < g.K) return NF4_ERR_ARG;
    for (int i = 0; i < nlora; ++i) {
        const nf4_lora &l = loras[i];
        if (l.seg < 0 || l.seg >= nw || l.rank < 1 || l.rank > 64 || !l.a || !l.da) return NF4_ERR_ARG;
        LoraDev &d = g.lora[l.seg];
        if (d.has) return NF4_ERR_ARG;
        d.a = static_cast<const uint16_t *>(l.a);
        d.da = static_cast<const uint16_t *>(l.da);
        d.rank = l.rank;
        d.scale = l.scale;
        d.has = 1;
    }
    if (m == 0 || g.K == 0) return NF4_OK;
    g.out = dx;
    g.ld_out = lddx;
    g.n_out = g.K;
    g.accumulate = accumulate != 0;
    g.vec_out = aligned(dx, 8) && lddx % 4 == 0;
    const Plan p = plan_dx(m, ws, nw);
    g.splits = p.splits;
    const int64_t bp = p.bp, bm = p.bm;
    g.m_tiles = (m + bm - 1) / bm;
    g.p_tiles = (g.K + bp - 1) / bp;
    g.step_start[0] = 0;
    for (int i = 0; i < nw; ++i) g.step_start[i + 1] = g.step_start[i] + (ws[i].rows + BR - 1) / BR;
    g.total_steps = g.step_start[nw];
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (p.splits > 1) {
        const size_t need = static_cast<size_t>(p.splits) * m * g.K * sizeof(float);
        if (!workspace || workspace_bytes < need) return NF4_ERR_WORKSPACE;
        g.partial = static_cast<float *>(workspace);
    }
    st = dtype == NF4_BF16 ? launch_dx<NF4_BF16>(g, p, s) : launch_dx<NF4_F16>(g, p, s);
    if (st != NF4_OK || p.splits <= 1) return st;
    return dtype == NF4_BF16 ? launch_reduce<NF4_BF16>(g, p.splits, s)
                             : launch_reduce<NF4_F16>(g, p.splits, s);
}
