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
// The 256x256 forward tile of a plain projection (fwd_body_rw) has each of its 8 waves own 32
// weight rows and dequantize them straight into its MFMA operand registers, only the
// activation tile going through LDS.  The other tilings stage both operands in LDS:
// workgroup tile BP x BM (256x256 with 8 waves, or 128x128 with 4), reduction step 64 (one NF4
// absmax block along k for the forward weight), two LDS stages and two register stages.  LDS
// tiles are rows of 64 16-bit values (128 bytes) whose 16-byte chunks are XOR-swizzled with bits
// 1..3 of the row, so the 16 rows one 16-lane group of an MFMA fragment read hit distinct banks.
// Per step s:
//   * activations and packed weight bytes of step s + 2 are loaded into registers through
//     buffer resources (hardware range checks return 0 past the end: no branches, so the
//     compiler's wait counts stay exact);
//   * the MFMAs of step s run in four k-substeps; after each substep a quarter of step s + 1's
//     staging runs: activation chunks to LDS, weight nibbles dequantized by a register table
//     (v_perm_b32 byte selects over the 16 values round(code[i] * absmax), absmax rebuilt from
//     its uint8 code) and written to LDS;
//   * one barrier.
// The dX weight tile keeps W's natural [n][k] layout; the MFMA A operand (rows k) is read
// transposed out of it with ds_read_b64_tr_b16.
// Long reductions are split over workgroups into fp32 partial sums that a reduction kernel
// adds up in a fixed order (deterministic).

#include <mutex>
#include <type_traits>

#include "nf4_common.h"

namespace {

constexpr int BR = 64;           // reduction step
constexpr int ROWB = 128;        // bytes per LDS tile row
constexpr int kMaxSeg = NF4_MAX_SEGMENTS;

// Byte offset of 16-byte chunk c (elements 8c..8c+7) of row r in an LDS tile.  gfx950's LDS
// serves a 16-byte-per-lane access 16 lanes (256 bytes, 64 banks) at a time; XOR-ing the chunk
// with bits 1..3 of the row makes the 16 rows such a group reads (an MFMA fragment: 16
// consecutive rows, one chunk) land on 16 distinct (row parity, chunk) bank slots.
__device__ __forceinline__ int swz(int r, int c) { return r * ROWB + ((c ^ ((r >> 1) & 7)) << 4); }

struct LoraDev {
    const uint16_t *t;   // forward: [M, rank]
    const uint16_t *b;   // forward: [rows_seg, rank]
    const uint16_t *a;   // dx: [rank, K]
    const uint16_t *da;  // dx: [M, rank]
    const uint16_t *xa;  // forward, computed in the launch: A [rank, K], and T = X A^T out to
    uint16_t *t_out;     //   t_out [M, rank] (skinny path, rank <= 16); else null
    float scale;
    int rank;
    int has;
    int vec;             // rank % 8 == 0 and 16-byte aligned rows: 16-byte fragment loads
};

// Tile decomposition of one part of a launch: tiles run segment by segment (forward) with m
// fastest; a two-part launch (head + tail plans) holds one map per part.
struct TileMap {
    int64_t m_tiles;
    int64_t tile_start[kMaxSeg + 1];  // forward: cumulative (p tiles x m tiles) per segment
    int64_t row0[kMaxSeg];            // forward: first row of each segment the part covers
    int64_t col0;                     // dx: first output column the part covers
};

struct GemmArgs {
    const uint16_t *act;          // X (forward) or dY (dx)
    int64_t ld_act;
    int64_t act_cols;             // valid columns of a row of act (forward: K; dx: sum rows)
    int64_t M;
    int64_t K;                    // in_features of every segment
    DevWeight w[kMaxSeg];
    int64_t seg_off[kMaxSeg];     // forward: output column offset; dx: dY column offset
    TileMap map[2];               // [1]: the second part of a two-part launch
    int64_t blocks0;              // two-part launch: workgroups of the first part (else 0)
    int64_t step_start[kMaxSeg + 1];  // dx: cumulative reduction steps per segment
    int nseg;
    LoraDev lora[kMaxSeg];
    const uint16_t *bias;         // forward: [sum rows] or null
    void *out;
    int64_t ld_out;
    int64_t n_out;                // forward: sum rows; dx: K
    // Tiles [0, tail_start) run whole; tiles [tail_start, tiles) (a column range
    // [tail_col0, n_out) of the output) are split over `splits` workgroups each, which write
    // fp32 partials [splits][M][tail_cols] for the fixed-order reduction kernel.
    float *partial;               // split workspace or null
    int splits;
    int64_t per_split;            // reduction steps per split (host-computed: no divisions)
    int64_t tail_start;
    int64_t tail_col0;
    int64_t tail_cols;
    int64_t total_steps;          // dx: sum of step counts
    int accumulate;               // dx: add into out
    int vec_out;                  // 8-byte output stores allowed (paired: and aux loads)
    const uint16_t *aux;          // paired SwiGLU backward: dH [M, I]
    int64_t ld_aux;
    int vec16_out;                // 16-byte output stores allowed (the LDS epilogue)
    int rows_groups;              // row-streaming path: row groups per workgroup
    int rows_parts;               // row-streaming path: K parts per row
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

// 16x16x32 MFMA: lane l holds row (A) / column (B) l % 16, k = 8 (l / 16) .. + 7; D lane l
// holds rows 4 (l / 16) .. + 3 of column l % 16.
template <int DT>
__device__ __forceinline__ float4_t mfma16(const u32x4_t &a, const u32x4_t &b, const float4_t &c) {
    if constexpr (DT == NF4_BF16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf168_t, a),
                                                      __builtin_bit_cast(bf168_t, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
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
    return round16<DT>(v);
}

__device__ __forceinline__ int seg_of_tile(const GemmArgs &a, const TileMap &tm, int64_t t) {
    int s = 0;
#pragma unroll
    for (int i = 1; i < kMaxSeg; ++i)
        if (i < a.nseg && t >= tm.tile_start[i]) s = i;
    return s;
}

__device__ __forceinline__ int seg_of_step(const GemmArgs &a, int64_t t) {
    int s = 0;
#pragma unroll
    for (int i = 1; i < kMaxSeg; ++i)
        if (i < a.nseg && t >= a.step_start[i]) s = i;
    return s;
}

// A value known to be the same in every lane, kept in scalar registers (the compiler otherwise
// can lose track through VALU-computed integer division and then wraps every buffer load that
// uses it in a per-lane loop).
__device__ __forceinline__ int64_t uniform64(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Tiles run m fastest: the dispatcher deals workgroups to the 8 XCDs in turn (XCD = id mod 8,
// each with its own L2), so with a multiple of 8 m tiles every XCD keeps the same m tiles and
// reads its share of the activations once, while the NF4 weight tiles (a quarter of the bytes
// per element) are read by every XCD.  Grouping a weight tile's m tiles on one XCD instead
// measured 2x the L2 miss bytes (every XCD then reads all the activations).
//
// Workgroup -> (tile, split, number of splits of that tile): 1-D grid of tail_start whole
// tiles followed by `splits` workgroups per tail tile.  32-bit arithmetic.
struct BlockTile {
    int64_t tile;
    int split;
    int nsplit;
};

__device__ __forceinline__ BlockTile block_tile(const GemmArgs &a, uint32_t b) {
    const uint32_t ts = static_cast<uint32_t>(a.tail_start);
    if (b < ts) return BlockTile{b, 0, 1};
    const uint32_t r = b - ts, sp = static_cast<uint32_t>(a.splits);
    return BlockTile{static_cast<int64_t>(__builtin_amdgcn_readfirstlane(ts + r / sp)),
                     static_cast<int>(__builtin_amdgcn_readfirstlane(r % sp)), a.splits};
}

// The raw absmax inputs of block b, fetched with the packed bytes; rebuilt later by absmax_val.
struct AbsIn {
    float s;      // absmax2 scale (nested) or the fp32 absmax
    uint32_t q;   // uint8 code (nested)
};

// Branch-free over the weight's format: the kernels' code2 tables hold {1, 0, ..} for a weight
// without double quantization, whose uint8 code reads 0 (empty resource), so 1 * s + 0 rebuilds
// the fp32 absmax s exactly (absmax >= 0: no -0 to lose).
__device__ __forceinline__ float code2_entry(const DevWeight &w, int i) {
    return w.nested ? w.code2[i] : (i == 0 ? 1.0f : 0.0f);
}

__device__ __forceinline__ float absmax_val(const DevWeight &w, const AbsIn &in, const float *code2) {
    return __fadd_rn(__fmul_rn(code2[in.q], in.s), w.nested ? w.offset : 0.0f);
}

// Resources of one weight: packed bytes, uint8 absmax codes (nested) and the fp32 scale array
// (absmax2 when nested, the fp32 absmax otherwise).
struct WeightRsrc {
    rsrc_t packed, q, s;
    int nested;
    int bs_shift, bs2_shift;
};

// (The fused kernels take power-of-two block sizes only: shifts, no 64-bit divisions.)
__device__ __forceinline__ WeightRsrc weight_rsrc(const DevWeight &w) {
    const int64_t n = w.rows * w.cols;
    const int64_t nb = (n + w.blocksize - 1) >> w.bs_shift;
    WeightRsrc r;
    r.packed = make_rsrc(w.packed, (n + 1) / 2);
    r.nested = w.nested;
    r.bs_shift = w.bs_shift;
    r.bs2_shift = w.bs2_shift;
    if (w.nested) {
        r.q = make_rsrc(w.absmax, nb);
        r.s = make_rsrc(w.absmax2, ((nb + w.blocksize2 - 1) >> w.bs2_shift) * 4);
    } else {
        r.q = make_rsrc(w.absmax, 0);
        r.s = make_rsrc(w.absmax, nb * 4);
    }
    return r;
}

// The absmax inputs of block b: uint8 code + absmax2 scale (nested) or the fp32 absmax.
__device__ __forceinline__ AbsIn absmax_bload(const WeightRsrc &r, int b) {
    AbsIn a;
    a.q = bload1(r.q, b);
    const int si = r.nested ? (b >> r.bs2_shift) : b;
    a.s = __builtin_bit_cast(float, bload4(r.s, si * 4));
    return a;
}

// ------------------------------------------------------------------ activation tile loader

// Per-thread byte offsets of an activation tile inside its window: thread t loads chunk t % 8
// (8 elements) of rows t / 8, t / 8 + NT / 8, ...; a step adds its column offset.  32-bit:
// the window is below 2 GiB.
struct ActAddr {
    int base;   // row t / 8, chunk t % 8
    int rstep;  // bytes between the rows one thread loads
};

template <int NT>
__device__ __forceinline__ ActAddr act_addr(int64_t ld) {
    ActAddr r;
    const int t = threadIdx.x % NT;
    r.base = static_cast<int>(((t >> 3) * ld + (t & 7) * 8) * 2);
    r.rstep = static_cast<int>((NT / 8) * ld * 2);
    return r;
}

// BM rows x 64 columns of act[m][col0 ..] staged through registers (the dX kernels' dY tile,
// whose partial steps are masked in registers; the forward tile goes by LDS DMA): load() issues the global
// loads of a step (16 bytes per chunk, 8 consecutive threads per 128-byte row), store() writes
// them to an LDS tile after the current step's MFMAs, so the wait for the loads lands there.
// Rows >= M read as zero.
template <int BM, int NT>
struct ActTile {
    static constexpr int CH = BM * 8 / NT;
    static_assert(CH >= 1 && BM * 8 % NT == 0, "tile rows must split evenly over the threads");
    u32x4_t r[CH];

    __device__ __forceinline__ void load(rsrc_t rs, const ActAddr &ad, int col_bytes) {
#pragma unroll
        for (int i = 0; i < CH; ++i) r[i] = bload16(rs, ad.base + i * ad.rstep + col_bytes);
    }

    // Zero the elements at columns >= valid of the step (a segment's partial last step).
    __device__ __forceinline__ void mask(int valid) {
        const int k = valid - static_cast<int>(threadIdx.x % NT & 7) * 8;  // valid elements of my chunks
        uint32_t mk[4];
#pragma unroll
        for (int d = 0; d < 4; ++d)
            mk[d] = ((2 * d < k) ? 0x0000ffffu : 0u) | ((2 * d + 1 < k) ? 0xffff0000u : 0u);
#pragma unroll
        for (int i = 0; i < CH; ++i)
            r[i] = (u32x4_t){r[i].x & mk[0], r[i].y & mk[1], r[i].z & mk[2], r[i].w & mk[3]};
    }

    __device__ __forceinline__ void store(uint8_t *s) const {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int idx = i * NT + threadIdx.x % NT;
            *reinterpret_cast<u32x4_t *>(s + swz(idx >> 3, idx & 7)) = r[i];
        }
    }

    // Chunks i with i % 4 == part (one quarter of the tile per MFMA k-substep).
    __device__ __forceinline__ void store_part(uint8_t *s, int part) const {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            if (i % 4 != part) continue;
            const int idx = i * NT + threadIdx.x % NT;
            *reinterpret_cast<u32x4_t *>(s + swz(idx >> 3, idx & 7)) = r[i];
        }
    }
};

// Resource over the BM-row activation window of a workgroup.
template <int BM>
__device__ __forceinline__ rsrc_t act_rsrc(const GemmArgs &a, int64_t m0) {
    const int64_t rows = a.M - m0 < BM ? a.M - m0 : BM;
    return make_rsrc(a.act + m0 * a.ld_act, ((rows - 1) * a.ld_act + a.act_cols) * 2);
}

// ------------------------------------------------------------------------- MFMA core

// LDS tile row of a wave's weight fragment i: consecutive 32-row fragments from prow0, or for a
// paired (gate | up) tile with halves of PH rows the first TP / 2 fragments from prow0 in the
// gate half and the last TP / 2 at the same rows of the up half.
template <int TP, int PH>
__device__ __forceinline__ int frag_row(int prow0, int i) {
    if constexpr (PH == 0) return prow0 + i * 32;
    else return i < TP / 2 ? prow0 + i * 32 : PH + prow0 + (i - TP / 2) * 32;
}

// Wave-level MFMA over one 64-deep step: acc[TP][TM] += Wop[p rows] x Act[m rows].
template <int DT, int TP, int TM, int PH = 0>
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
            fa[i] = *reinterpret_cast<const u32x4_t *>(sw + swz(frag_row<TP, PH>(prow0, i) + r, c));
#pragma unroll
        for (int j = 0; j < TM; ++j)
            fb[j] = *reinterpret_cast<const u32x4_t *>(sa + swz(mrow0 + j * 32 + r, c));
#pragma unroll
        for (int i = 0; i < TP; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) acc[i][j] = mfma32<DT>(fa[i], fb[j], acc[i][j]);
    }
}

// mma_step with part ks of the next tile's staging work (`part(ks)`: global-to-LDS copy and
// dequantization of data already in registers) placed among the MFMAs of k-substep ks, so the
// VALU and LDS-write work runs while the matrix unit is busy.
template <int DT, int TP, int TM, int PH = 0, class Part>
__device__ __forceinline__ void mma_step_interleaved(float16_t (&acc)[TP][TM], const uint8_t *sw,
                                                     const uint8_t *sa, int prow0, int mrow0,
                                                     Part &&part) {
    const int lane = threadIdx.x & 63;
    const int r = lane & 31;
    const int kh = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < BR / 16; ++ks) {
        const int c = ks * 2 + kh;
        u32x4_t fa[TP], fb[TM];
#pragma unroll
        for (int i = 0; i < TP; ++i)
            fa[i] = *reinterpret_cast<const u32x4_t *>(sw + swz(frag_row<TP, PH>(prow0, i) + r, c));
#pragma unroll
        for (int j = 0; j < TM; ++j)
            fb[j] = *reinterpret_cast<const u32x4_t *>(sa + swz(mrow0 + j * 32 + r, c));
#pragma unroll
        for (int i = 0; i < TP; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) acc[i][j] = mfma32<DT>(fa[i], fb[j], acc[i][j]);
        part(ks);
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

// 8 consecutive 16-bit values of a LoRA row (src[0 .. lim)): one 16-byte load when the rows
// allow it (`vec`), else element by element.
__device__ __forceinline__ u32x4_t lora_row8(const uint16_t *src, int lim, int vec) {
    if (vec && lim >= 8) return *reinterpret_cast<const u32x4_t *>(src);
    return gather8(src, 1, lim);
}

// Epilogue: lane holds C[p .. p+3][m] for each (i, j, r4).  Writes either fp32 partials
// (a split tail tile) or final values (+bias, +existing for accumulate) in DT.  With KG k-groups
// in the workgroup, group g writes the fragments j with j % KG == g (see group_sum).
template <int DT, int TP, int TM, int KG = 1>
__device__ __forceinline__ void epilogue(const GemmArgs &a, float16_t (&acc)[TP][TM],
                                         int64_t p_base, int64_t p_end, int64_t col_off,
                                         int64_t m_base, int split, bool to_partial, int g = 0) {
    const int lane = threadIdx.x & 63;
    // fragments j inside (i, r4): a lane's columns are the same in every j, so their bias is
    // loaded once per (i, r4)
#pragma unroll
    for (int i = 0; i < TP; ++i) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int64_t p = p_base + i * 32 + r4 * 8 + (lane >> 5) * 4;
            if (p >= p_end) continue;
            const int64_t col = col_off + p;
            const bool full = p + 4 <= p_end;
            float bv[4] = {0.f, 0.f, 0.f, 0.f};
            if (a.bias && !to_partial) {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (p + q < p_end) bv[q] = to_f32<DT>(a.bias[col + q]);
            }
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                if (KG > 1 && j % KG != g) continue;  // another k-group's fragments
                const int64_t m = m_base + j * 32 + (lane & 31);
                if (m >= a.M) continue;
                float v[4] = {acc[i][j][r4 * 4 + 0], acc[i][j][r4 * 4 + 1],
                              acc[i][j][r4 * 4 + 2], acc[i][j][r4 * 4 + 3]};
                if (to_partial) {
                    float *dst = a.partial + (static_cast<int64_t>(split) * a.M + m) * a.tail_cols +
                                 (col - a.tail_col0);
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
                    for (int q = 0; q < 4; ++q) v[q] += bv[q];
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

// Epilogue of an unsplit tile without a bias or an accumulated output through LDS: the
// finished values are rounded to the output dtype and written to LDS in the output's row-major
// layout, then stored as whole 16-byte chunks, one thread per chunk of a tile row (with
// k-groups each group writes the fragments it finished and every thread of the workgroup
// stores).  Stored straight
// from the MFMA layout, each 8-byte store instruction would touch 32 output rows with 16 bytes
// each (128 KB per 256x256 tile in 8192 pieces): measured 10-17 % of a K = 1536 launch, against
// ~5 % this way.  LDS row m (one output row of the tile) holds its BP columns as BP / 8 chunks of
// 8 values, chunk c at position c ^ (m % min(32, BP / 8)), so the rows one MFMA fragment's lanes
// write hit distinct chunks (two lanes per chunk for BP = 128).  Uses the staging LDS (BM x 2 BP
// bytes) after every wave's last fragment read.
template <int DT, int BP, int BM, int TP, int TM, int NT, int KG = 1>
__device__ __forceinline__ void epilogue_lds(const GemmArgs &a, float16_t (&acc)[TP][TM],
                                             uint8_t *lds, int64_t p0, int prow0, int64_t p_end,
                                             int64_t col_off, int64_t m0, int mrow0, int g = 0) {
    constexpr int RB = BP * 2;           // bytes of a tile row in LDS
    constexpr int CPR = BP / 8;          // 16-byte chunks per row
    constexpr int SW = CPR < 32 ? CPR : 32;
    const int lane = threadIdx.x & 63;
    __syncthreads();  // every wave's last fragment reads (and k-group sums) are done
    // Group g writes fragments j = KG jj + g.  The fragment is picked by selects rather than
    // by a branch on g, which the compiler turns into dynamic indexing of acc (a copy of the
    // accumulators in scratch memory).
#pragma unroll
    for (int jj = 0; jj < TM / KG; ++jj) {
        const int m = mrow0 + (jj * KG + g) * 32 + (lane & 31);
#pragma unroll
        for (int i = 0; i < TP; ++i) {
            float16_t v = acc[i][jj * KG];
#pragma unroll
            for (int q = 1; q < KG; ++q)
                if (g == q) v = acc[i][jj * KG + q];
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int p = prow0 + i * 32 + r4 * 8 + (lane >> 5) * 4;  // tile column
                u32x2_t o;
                o.x = pack2<DT>(v[r4 * 4 + 0], v[r4 * 4 + 1]);
                o.y = pack2<DT>(v[r4 * 4 + 2], v[r4 * 4 + 3]);
                const int c = (p >> 3) ^ (m & (SW - 1));
                *reinterpret_cast<u32x2_t *>(lds + m * RB + c * 16 + (p & 7) * 2) = o;
            }
        }
    }
    __syncthreads();
    constexpr int NTA = KG * NT;  // every thread of the workgroup stores
    const int t = threadIdx.x % NTA;
    const int c = t % CPR;  // the thread's chunk of a row: columns 8c .. 8c + 7
    constexpr int RSTEP = NTA / CPR;  // tile rows stored per pass
    static_assert(BM % RSTEP == 0, "whole passes over the tile rows");
#pragma unroll 4
    for (int it = 0; it < BM / RSTEP; ++it) {
        const int m = t / CPR + it * RSTEP;
        const int64_t gm = m0 + m;
        const int64_t p = p0 + 8 * c;
        if (gm >= a.M || p >= p_end) continue;
        u32x4_t v = *reinterpret_cast<const u32x4_t *>(lds + m * RB + ((c ^ (m & (SW - 1))) << 4));
        uint16_t *dst = static_cast<uint16_t *>(a.out) + gm * a.ld_out + col_off + p;
        if (p + 8 > p_end) {  // the last, partial chunk of a row
            const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (p + e < p_end) dst[e] = static_cast<uint16_t>(wv[e >> 1] >> ((e & 1) * 16));
            continue;
        }
        *reinterpret_cast<u32x4_t *>(dst) = v;
    }
}

// epilogue_lds for tiles with a bias or an accumulated output: the accumulators go to LDS as
// fp32 (BM x BP x 4 bytes, chunk cc = 4 columns of row m at cc ^ (m % 32)), and the bias and
// the existing output are added in fp32 before the one rounding, in the order of the
// register epilogue (bit-identical to it).  Each thread's 8 columns are the same on every row
// it stores, so it loads their bias once.
template <int DT, int BP, int BM, int TP, int TM, int NT, int KG = 1>
__device__ __forceinline__ void epilogue_lds32(const GemmArgs &a, float16_t (&acc)[TP][TM],
                                               uint8_t *lds, int64_t p0, int prow0, int64_t p_end,
                                               int64_t col_off, int64_t m0, int mrow0, int g = 0) {
    static_assert(BP / 4 == 32, "32 four-column chunks per LDS row");
    constexpr int RB = BP * 4;
    const int lane = threadIdx.x & 63;
    __syncthreads();  // every wave's last fragment reads (and k-group sums) are done
#pragma unroll
    for (int jj = 0; jj < TM / KG; ++jj) {
        const int m = mrow0 + (jj * KG + g) * 32 + (lane & 31);
#pragma unroll
        for (int i = 0; i < TP; ++i) {
            float16_t v = acc[i][jj * KG];
#pragma unroll
            for (int q = 1; q < KG; ++q)
                if (g == q) v = acc[i][jj * KG + q];
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int p = prow0 + i * 32 + r4 * 8 + (lane >> 5) * 4;
                *reinterpret_cast<float4_t *>(lds + m * RB + (((p >> 2) ^ (m & 31)) << 4)) =
                    (float4_t){v[r4 * 4], v[r4 * 4 + 1], v[r4 * 4 + 2], v[r4 * 4 + 3]};
            }
        }
    }
    __syncthreads();
    constexpr int NTA = KG * NT;
    constexpr int CPR = BP / 8;
    const int t = threadIdx.x % NTA;
    const int c = t % CPR;  // columns 8c .. 8c + 7: LDS chunks 2c and 2c + 1
    const int64_t p = p0 + 8 * c;
    float bf[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
        bf[e] = (a.bias && p + e < p_end) ? to_f32<DT>(a.bias[col_off + p + e]) : 0.0f;
    constexpr int RSTEP = NTA / CPR;
    static_assert(BM % RSTEP == 0, "whole passes over the tile rows");
#pragma unroll 2
    for (int it = 0; it < BM / RSTEP; ++it) {
        const int m = t / CPR + it * RSTEP;
        const int64_t gm = m0 + m;
        if (gm >= a.M || p >= p_end) continue;
        const float4_t lo4 = *reinterpret_cast<const float4_t *>(lds + m * RB + (((2 * c) ^ (m & 31)) << 4));
        const float4_t hi4 = *reinterpret_cast<const float4_t *>(lds + m * RB + (((2 * c + 1) ^ (m & 31)) << 4));
        float f[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
        if (a.bias) {
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] += bf[e];
        }
        uint16_t *dst = static_cast<uint16_t *>(a.out) + gm * a.ld_out + col_off + p;
        if (p + 8 > p_end) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (p + e < p_end) {
                    float x = f[e];
                    if (a.accumulate) x += to_f32<DT>(dst[e]);
                    dst[e] = from_f32<DT>(x);
                }
            continue;
        }
        if (a.accumulate) {
            const u32x4_t old = *reinterpret_cast<const u32x4_t *>(dst);
            const uint32_t ow[4] = {old.x, old.y, old.z, old.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                f[2 * e] += to_f32<DT>(ow[e] & 0xffff);
                f[2 * e + 1] += to_f32<DT>(ow[e] >> 16);
            }
        }
        *reinterpret_cast<u32x4_t *>(dst) = (u32x4_t){pack2<DT>(f[0], f[1]), pack2<DT>(f[2], f[3]),
                                                      pack2<DT>(f[4], f[5]), pack2<DT>(f[6], f[7])};
    }
}

// The split-K partial sums of a 256-wide tile the same way, in fp32: the 256 x 256 tile is
// 256 KB, so it goes through the staging LDS in two halves of 128 rows m (a wave's rows lie in
// one half); LDS row m holds 256 floats as 64 chunks of 4, chunk c at c ^ (m % 32).
template <int BM, int WM, int TP, int TM, int NT>
__device__ __forceinline__ void partial_lds(const GemmArgs &a, float16_t (&acc)[TP][TM],
                                            uint8_t *lds, int64_t p0, int prow0, int64_t p_end,
                                            int64_t col_off, int64_t m0, int mrow0, int split) {
    static_assert(BM % 128 == 0, "whole halves of 128 rows");
    const int lane = threadIdx.x & 63;
    const int t = threadIdx.x % NT;
    const int c = t & 63;  // the thread's chunk of a row: columns 4c .. 4c + 3
#pragma unroll 1
    for (int h = 0; h < BM / 128; ++h) {
        __syncthreads();  // the staging tiles (h = 0) or the previous half's reads are done
        {
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                if ((mrow0 + j * 32) / 128 != h) continue;  // the fragment lies in the other half
                const int m = mrow0 - 128 * h + j * 32 + (lane & 31);
#pragma unroll
                for (int i = 0; i < TP; ++i)
#pragma unroll
                    for (int r4 = 0; r4 < 4; ++r4) {
                        const int p = prow0 + i * 32 + r4 * 8 + (lane >> 5) * 4;
                        const int cc = (p >> 2) ^ (m & 31);
                        *reinterpret_cast<float4_t *>(lds + m * 1024 + cc * 16) =
                            (float4_t){acc[i][j][r4 * 4 + 0], acc[i][j][r4 * 4 + 1],
                                       acc[i][j][r4 * 4 + 2], acc[i][j][r4 * 4 + 3]};
                    }
            }
        }
        __syncthreads();
#pragma unroll 4
        for (int m = t >> 6; m < 128; m += NT / 64) {
            const int64_t gm = m0 + 128 * h + m;
            const int64_t p = p0 + 4 * c;
            if (gm >= a.M || p >= p_end) continue;
            const float4_t v = *reinterpret_cast<const float4_t *>(lds + m * 1024 + ((c ^ (m & 31)) << 4));
            float *dst = a.partial + (static_cast<int64_t>(split) * a.M + gm) * a.tail_cols +
                         (col_off + p - a.tail_col0);
            if (p + 4 <= p_end) {
                *reinterpret_cast<float4_t *>(dst) = v;
            } else {
                for (int e = 0; e < 4; ++e)
                    if (p + e < p_end) dst[e] = v[e];
            }
        }
    }
}

// ------------------------------------------------------------------------ weight tiles

// Forward weight tile: BP rows x 64 k of W (natural layout).  Thread t owns 16 packed bytes =
// 32 elements of row t/2 (one absmax); NT == 2 * BP.  Offsets are 32-bit: a weight with one
// tile of rows past its end stays below 2 GiB (checked on the host).
struct WAddr {
    int packed;  // byte offset of this thread's 16 packed bytes at step 0
    int block;   // absmax block of this thread's row at step 0
};

template <int BP>
__device__ __forceinline__ WAddr fwd_waddr(const WeightRsrc &r, int64_t p0, int64_t K) {
    const int t = threadIdx.x % (2 * BP);
    const int64_t row = p0 + (t >> 1);
    WAddr a;
    a.packed = static_cast<int>(row * (K >> 1) + (t & 1) * 16);
    a.block = static_cast<int>(row * (K >> r.bs_shift));
    return a;
}

template <int DT, int BP>
struct FwdWeight {
    u32x4_t raw;
    AbsIn abs;

    // Rows past the weight read as zero (their outputs are never stored).
    __device__ __forceinline__ void load(const WeightRsrc &r, const WAddr &ad, int64_t st) {
        raw = bload16(r.packed, ad.packed + static_cast<int>(st) * (BR / 2));
        abs = absmax_bload(r, ad.block + static_cast<int>((st * BR) >> r.bs_shift));
    }

    // Dword `part` of the 16 packed bytes (8 elements) through the register table of this
    // thread's row: the half table (make_table_half) that this thread and its partner, the other
    // half of the row's 64-deep step (thread t ^ 1), build together.
    __device__ __forceinline__ void store_part(uint8_t *s, const Nf4Table &tb, uint32_t selbase,
                                               int part) const {
        const int t = threadIdx.x % (2 * BP);
        const int row = t >> 1, h = (t & 1) * 4;
        const uint32_t wd = part == 0 ? raw.x : part == 1 ? raw.y : part == 2 ? raw.z : raw.w;
        *reinterpret_cast<u32x4_t *>(s + swz(row, h + part)) = lookup8s(tb, wd, selbase);
    }
};

// dX weight tile: 64 rows n x BP columns k of W in its natural layout (rows of BP 16-bit values,
// 16-byte chunks c swizzled by swz_t).  Thread t dequantizes 32 consecutive k of row
// t / (BP / 32): one absmax, one register table, four 16-byte LDS writes, as the forward tile.
// The MFMA reads it transposed (mma_step_dx below).
//
// Rows start on bank 0 (256 or 512 bytes), so the bank group of a chunk is its index mod 16, and
// LDS serves 16 lanes of a 16-byte access per pass.  A store pass covers chunks 4j + part of
// two rows (j < 8, BP = 256) or of four rows (j < 4, BP = 128); a transposed read pass covers
// chunks c0 .. c0 + 3 of rows n0 .. n0 + 3 (c0, n0 multiples of 4).  Chunk c of row n goes to
// c ^ 4 (n & 3) ^ low, where the low two bits separate what the store passes share: c / 16 and
// row parity for BP = 256, the row mod 4 for BP = 128.  Every pass then hits 16 distinct bank
// groups (the reads: 4 (n & 3) keeps the rows apart, low only permutes a row's 4 chunks).
template <int BP>
__device__ __forceinline__ int swz_t(int n, int c) {
    const int low = BP == 256 ? (((c >> 4) & 1) ^ ((n & 1) << 1)) : (n & 3);
    return n * (BP * 2) + ((c ^ ((n & 3) << 2) ^ low) << 4);
}

template <int BP>
__device__ __forceinline__ WAddr dx_waddr(const WeightRsrc &r, int64_t p0, int64_t K) {
    constexpr int KQ = BP / 32;
    const int t = threadIdx.x % (2 * BP);
    const int64_t n = t / KQ, k = p0 + (t % KQ) * 32;
    WAddr a;
    a.packed = static_cast<int>((n * K + k) >> 1);
    a.block = static_cast<int>(n * (K >> r.bs_shift) + (k >> r.bs_shift));
    return a;
}

template <int DT, int BP>
struct DxWeight {
    static constexpr int KQ = BP / 32;   // threads per tile row
    u32x4_t raw;
    AbsIn abs;

    // Step n0 (segment-local row of the step's first n): rows past the segment read as zero;
    // columns past K read neighbouring bytes (their outputs are never stored).
    __device__ __forceinline__ void load(const WeightRsrc &r, const WAddr &ad, int64_t n0, int64_t K) {
        raw = bload16(r.packed, ad.packed + static_cast<int>(n0 * (K >> 1)));
        abs = absmax_bload(r, ad.block + static_cast<int>(n0 * (K >> r.bs_shift)));
    }

    // through the half table shared with thread t ^ 1 (the other 32 k of the same absmax block)
    __device__ __forceinline__ void store_part(uint8_t *s, const Nf4Table &tb, uint32_t selbase,
                                               int part) const {
        const int t = threadIdx.x % (2 * BP);
        const int n = t / KQ, c = (t % KQ) * 4 + part;
        const uint32_t wd = part == 0 ? raw.x : part == 1 ? raw.y : part == 2 ? raw.z : raw.w;
        *reinterpret_cast<u32x4_t *>(s + swz_t<BP>(n, c)) = lookup8s(tb, wd, selbase);
    }
};

// dX MFMA step: A operand = W^T (rows k) read transposed from the natural-layout tile with
// ds_read_b64_tr_b16: in each 16-lane group, lane q points at 4 consecutive k of row
// n0 + q / 4, and lane q then holds W[n0 .. n0+3][k0 + q]; two reads give the 8 n of a
// 32x32x16 fragment.  B operand = dY tile (rows m) as in the forward kernel.
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

__device__ __forceinline__ uint2 tr_read(const uint8_t *s, int off) {
    const v4i16_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4i16_t *)((__attribute__((address_space(3))) uint8_t *)s + off));
    return __builtin_bit_cast(uint2, v);
}

template <int DT, int BP, int TP, int TM, class Part>
__device__ __forceinline__ void mma_step_dx(float16_t (&acc)[TP][TM], const uint8_t *sw,
                                            const uint8_t *sa, int prow0, int mrow0, Part &&part) {
    const int lane = threadIdx.x & 63;
    const int r = lane & 31;
    const int kh = lane >> 5;
    const int q = lane & 15, g = lane >> 4;
#pragma unroll
    for (int ks = 0; ks < BR / 16; ++ks) {
        u32x4_t fa[TP], fb[TM];
        const int n0 = ks * 16 + (g >> 1) * 8 + (q >> 2);
#pragma unroll
        for (int i = 0; i < TP; ++i) {
            const int k = prow0 + i * 32 + (g & 1) * 16 + (q & 3) * 4;
            const uint2 lo = tr_read(sw, swz_t<BP>(n0, k >> 3) + (k & 7) * 2);
            const uint2 hi = tr_read(sw, swz_t<BP>(n0 + 4, k >> 3) + (k & 7) * 2);
            fa[i] = (u32x4_t){lo.x, lo.y, hi.x, hi.y};
        }
#pragma unroll
        for (int j = 0; j < TM; ++j)
            fb[j] = *reinterpret_cast<const u32x4_t *>(sa + swz(mrow0 + j * 32 + r, ks * 2 + kh));
#pragma unroll
        for (int i = 0; i < TP; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) acc[i][j] = mfma32<DT>(fa[i], fb[j], acc[i][j]);
        part(ks);
    }
}

// SwiGLU epilogue of a paired (gate | up) tile: fragments i < TP / 2 hold gate rows j and
// fragments i + TP / 2 the same up rows, so a lane holds g and u of the same (m, j).
//   forward:  H[m][j] = silu(g) u                                 (out [M, I])
//   backward: dG[m][j] = dH u silu'(g), dU[m][j] = dH silu(g)     (out [M, 2I]: dG | dU)
// with silu'(g) = sig (1 + g (1 - sig)), sig = 1 / (1 + exp(-g)), the standalone SwiGLU
// kernels' formulas applied to the fp32 accumulators instead of rounded g and u; the reciprocal
// is the hardware's (1 ulp) instead of a correctly rounded division: the epilogue runs after
// each tile's main loop, where a dozen-instruction division per element shows.  The dH loads
// of a lane are all issued before its first use.
template <int DT, int TP, int TM, bool BWD, int KG = 1>
__device__ __forceinline__ void epilogue_swiglu(const GemmArgs &a, float16_t (&acc)[TP][TM],
                                                int64_t j_base, int64_t n_inter, int64_t m_base,
                                                int g = 0) {
    const int lane = threadIdx.x & 63;
    // dH of every (m, 4 j) group of the lane, loaded before any is used (zero outside)
    u32x2_t dhv[TM][TP / 2][4];
    if constexpr (BWD) {
#pragma unroll
        for (int jm = 0; jm < TM; ++jm) {
            if (KG > 1 && jm % KG != g) continue;
            const int64_t m = m_base + jm * 32 + (lane & 31);
#pragma unroll
            for (int i = 0; i < TP / 2; ++i)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int64_t j = j_base + i * 32 + r4 * 8 + (lane >> 5) * 4;
                    u32x2_t v = {0u, 0u};
                    if (m < a.M && j < n_inter) {
                        const uint16_t *src = a.aux + m * a.ld_aux + j;
                        if (j + 4 <= n_inter && a.vec_out) {
                            v = *reinterpret_cast<const u32x2_t *>(src);
                        } else {
                            uint32_t e[4] = {0u, 0u, 0u, 0u};
                            for (int q = 0; q < 4; ++q)
                                if (j + q < n_inter) e[q] = src[q];
                            v = (u32x2_t){e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
                        }
                    }
                    dhv[jm][i][r4] = v;
                }
        }
    }
#pragma unroll
    for (int jm = 0; jm < TM; ++jm) {
        if (KG > 1 && jm % KG != g) continue;
        const int64_t m = m_base + jm * 32 + (lane & 31);
        if (m >= a.M) continue;
#pragma unroll
        for (int i = 0; i < TP / 2; ++i) {
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int64_t j = j_base + i * 32 + r4 * 8 + (lane >> 5) * 4;
                if (j >= n_inter) continue;
                const bool full = j + 4 <= n_inter && a.vec_out;
                float dh[4] = {0.f, 0.f, 0.f, 0.f};
                if constexpr (BWD) {
                    const u32x2_t v = dhv[jm][i][r4];
                    dh[0] = to_f32<DT>(v.x & 0xffff);
                    dh[1] = to_f32<DT>(v.x >> 16);
                    dh[2] = to_f32<DT>(v.y & 0xffff);
                    dh[3] = to_f32<DT>(v.y >> 16);
                }
                float o0[4], o1[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float g = acc[i][jm][r4 * 4 + q], u = acc[i + TP / 2][jm][r4 * 4 + q];
                    const float sig = __builtin_amdgcn_rcpf(1.0f + __expf(-g));
                    if constexpr (BWD) {
                        o0[q] = dh[q] * u * sig * (1.0f + g * (1.0f - sig));
                        o1[q] = dh[q] * g * sig;
                    } else {
                        o0[q] = g * sig * u;
                    }
                }
                uint16_t *dst = static_cast<uint16_t *>(a.out) + m * a.ld_out + j;
#pragma unroll
                for (int h = 0; h < (BWD ? 2 : 1); ++h) {
                    const float *v = h == 0 ? o0 : o1;
                    uint16_t *d = dst + h * n_inter;
                    if (full) {
                        u32x2_t o;
                        o.x = pack2<DT>(v[0], v[1]);
                        o.y = pack2<DT>(v[2], v[3]);
                        *reinterpret_cast<u32x2_t *>(d) = o;
                    } else {
                        for (int q = 0; q < 4; ++q)
                            if (j + q < n_inter) d[q] = from_f32<DT>(v[q]);
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------- kernels

// k-groups: a workgroup of KG groups of WP x WM waves; group g takes the steps s0 + g,
// s0 + g + KG, .. of the workgroup's reduction range through LDS stages of its own, with every
// group running the same number of steps (a group past the range runs its last step on zero
// activations), so that all waves meet at the same barriers.  Afterwards the groups add their
// accumulators through LDS: group g finishes the fragments j with j % KG == g and receives the
// other groups' values for those (one 16-byte slot per lane, 1 KB per wave instruction).  For
// KG = 2 the sum of the two groups is the same in either order.
template <int TP, int TM, int KG, int NT>
__device__ __forceinline__ void group_sum(float16_t (&acc)[TP][TM], uint8_t *lds, int g) {
    static_assert(KG == 2 && TM % 2 == 0, "two k-groups over an even number of m fragments");
    const int gt = threadIdx.x % NT;  // thread inside its group
    constexpr int ngt = NT;
    float4_t *slot = reinterpret_cast<float4_t *>(lds);
    __syncthreads();  // every group's last MFMAs have read the staging tiles
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        if (j % KG == g) continue;
#pragma unroll
        for (int i = 0; i < TP; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                slot[((j * TP + i) * 4 + q) * ngt + gt] =
                    (float4_t){acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                               acc[i][j][4 * q + 3]};
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        if (j % KG != g) continue;
#pragma unroll
        for (int i = 0; i < TP; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4_t v = slot[((j * TP + i) * 4 + q) * ngt + gt];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v[e];
            }
    }
}

// EPI 0: Y = X W^T (+ bias, + LoRA), split-K tails allowed.  EPI 1 / 2: paired gate | up
// tiles (segments 0 and 1, equal shapes) with the SwiGLU forward / backward epilogue: a tile
// covers BP / 2 rows j of both weights, gate in the first half of its W tile (dequantized by
// the first half of the waves) and up in the second, no bias, LoRA or split.  KG k-groups
// (group_sum above) split each tile's reduction inside the workgroup.
template <int BP, int BM, int KG>
constexpr int stage_bytes() {  // LDS of the staging tiles: KG groups x 2 stages x (W + act)
    return KG * 2 * (BP + BM) * ROWB;
}

// One workgroup of the forward GEMM: block `blk` of part `tm` of the launch, staging tiles in
// `lds` (stage_bytes<BP, BM, KG>() bytes), code2 tables in `s_code2`.
template <int DT, int BP, int BM, int WP, int WM, int EPI, int KG>
__device__ __forceinline__ void fwd_body(const GemmArgs &a, const TileMap &tm, uint32_t blk,
                                         uint8_t *lds, float (*s_code2)[256]) {
    constexpr int NT = WP * WM * 64;  // threads of one k-group
    constexpr int TP = BP / WP / 32, TM = BM / WM / 32;
    constexpr bool PAIR = EPI != 0;
    constexpr int PH = PAIR ? BP / 2 : 0;
    static_assert(NT == 2 * BP, "forward weight tile mapping needs 2 threads per row");
    static_assert(!PAIR || TP % 2 == 0, "paired tiles split each wave's fragments in halves");
    constexpr int NS = 2;  // LDS stages per k-group
    static_assert(KG == 1 || BP * BM * 4 <= stage_bytes<BP, BM, KG>(),
                  "the k-group sums fit in the staging tiles");
    auto sT = reinterpret_cast<uint8_t(*)[NS][(BP + BM) * ROWB]>(lds);

    // tiles: segments in order, m fastest.  32-bit tile arithmetic: 64-bit divisions are long
    // scalar sequences the whole CU waits on.
    const BlockTile bt = block_tile(a, blk);
    const int split = bt.split;
    const int64_t tile = bt.tile;
    const int seg = PAIR ? 0 : seg_of_tile(a, tm, tile);
    const uint32_t local = static_cast<uint32_t>(tile - tm.tile_start[seg]);
    const uint32_t mtl = static_cast<uint32_t>(tm.m_tiles);
    const int64_t p0 =
        uniform64(tm.row0[seg] + static_cast<int64_t>(local / mtl) * (PAIR ? PH : BP));
    const int64_t m0 = uniform64(static_cast<int64_t>(local % mtl) * BM);
    const int wave_all = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int g = KG > 1 ? wave_all / (WP * WM) : 0;           // k-group
    const int wave = KG > 1 ? wave_all % (WP * WM) : wave_all;  // wave inside the group
    // the weight this thread dequantizes (paired: the waves of W tile rows >= PH take up)
    const int wseg = PAIR ? (wave >= BP / 64 ? 1 : 0) : seg;
    const DevWeight w = a.w[wseg];  // by value: kept in registers for the whole loop
    const int64_t K = a.K;
    const int64_t steps = K / BR;
    const int64_t per = bt.nsplit > 1 ? a.per_split : steps;
    const int64_t s0 = uniform64(split * per);
    const int64_t s1 = uniform64(s0 + per < steps ? s0 + per : steps);
    // this group's steps: s0 + g + KG v for v < nv (the same nv in every group)
    const int64_t nv = (s1 - s0 + KG - 1) / KG;

    // code2 table entry threadIdx.x (every workgroup has at least 256 threads): loaded here,
    // written to LDS after the first two steps' loads and the LoRA slab's are issued, so that
    // their latency is not behind this load's
    // (buffer loads with no branch: threads past entry 255, and weights without nested
    // absmax, read zero)
    static_assert(KG * NT >= 256, "one code2 entry per thread");
    const int ci = static_cast<int>(threadIdx.x);
    const uint32_t c2a = bload4(make_rsrc(a.w[seg].code2, a.w[seg].nested ? 1024 : 0), ci * 4);
    const uint32_t c2b = PAIR ? bload4(make_rsrc(a.w[1].code2, a.w[1].nested ? 1024 : 0), ci * 4) : 0u;
    const float *code2 = s_code2[PAIR ? wseg : 0];
    float code_r[16];
    load_code_sgpr(w.code, code_r);
    const Nf4HalfCodes hc = half_codes(code_r);

    const int wp = wave % WP, wm = wave / WP;
    const int lane = threadIdx.x & 63;
    const int prow0 = wp * ((PAIR ? PH : BP) / WP);  // first W tile row of this wave's fragments

    float16_t acc[TP][TM];
#pragma unroll
    for (int i = 0; i < TP; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = (float16_t){};

    // Two LDS stages (steps v and v+1, in the group's step numbering v) and two weight register
    // stages.  Step v computes from LDS stage v & 1 while the other LDS stage receives step v+1:
    // its weights from register stage (v + 1) & 1, dequantized a quarter per MFMA k-substep, and
    // its activations straight from global memory by gfx950's 16-byte LDS DMA
    // (buffer_load_dwordx4 ... lds: lane i of the wave writes M0 + 16 i), issued after the
    // first quarter, when the weight registers of v+1 have been consumed; the global loads of
    // the weights of v+2 go out with it.  Wave w of a group fills the 8-row blocks CHA w ..
    // CHA w + CHA - 1 of the activation tile, lane i's source chunk chosen so that the block
    // lands in swz()'s layout (row r, position q holds chunk q ^ ((r >> 1) & 7)).  The loop
    // body has no branches: prefetches past the range are issued anyway (in bounds of the
    // operands or zero from the buffer range check, never consumed).  An odd last step runs
    // after the loop.  Rows past M, and a group's step past the workgroup's range (KG > 1 only,
    // an empty resource), read zeros.  The first two steps' loads are issued before the LoRA
    // slab and the table barrier, so that their latency overlaps the slab's loads.
    FwdWeight<DT, BP> wt[2] = {};
    const WeightRsrc wr = weight_rsrc(w);
    const rsrc_t ar = act_rsrc<BM>(a, m0);
    const rsrc_t ar0 = make_rsrc(a.act, 0);
    const WAddr wa = fwd_waddr<BP>(wr, p0 - (wseg == 1 ? PH : 0), K);
    constexpr int CHA = BM * 8 / NT;
    static_assert(CHA >= 1 && BM * 8 % NT == 0, "activation rows split evenly over the waves");
    int adoff[CHA];
#pragma unroll
    for (int j = 0; j < CHA; ++j) {
        const int row = (wave * CHA + j) * 8 + (lane >> 3);
        adoff[j] = row * static_cast<int>(a.ld_act) * 2 + (((lane & 7) ^ ((row >> 1) & 7)) << 4);
    }
    const uint32_t lds_a =  // this wave's activation rows in the group's LDS stage 0
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t *)lds)) +
        (g * NS * (BP + BM) + BP + wave * CHA * 8) * ROWB;
    // The DMA as inline assembly: the compiler does not count these loads, so none of its own
    // waits (for the weight registers) also waits for them; wait_dma() waits for them instead.
    // M0 is declared clobbered (hipcc notes that it is a reserved register): nothing else in
    // these kernels uses M0, so no value of the compiler's lives in it across the statement.
    auto dma_a = [&](int b, int64_t v) {  // activations of step v into LDS stage b
        const int64_t st = s0 + g + KG * v;
        const rsrc_t rs = KG > 1 && st >= s1 ? ar0 : ar;
        const int kb = static_cast<int>(st) * (BR * 2);
        const uint32_t base = __builtin_amdgcn_readfirstlane(lds_a + b * (BP + BM) * ROWB);
#pragma unroll
        for (int j = 0; j < CHA; ++j) {
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                         :
                         : "s"(base + j * 8 * ROWB), "v"(adoff[j]), "s"(rs), "s"(kb)
                         : "memory", "m0");
        }
    };
    // Every DMA is followed by exactly the 3 global loads of one weight register stage (packed
    // bytes, absmax code, absmax scale) and by nothing else before this wait, and loads complete
    // in order: vmcnt(3) has this wave's DMA in LDS.
    auto wait_dma = [] { asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); };
    auto stage = [&](int b, int64_t v) { wt[b].load(wr, wa, s0 + g + KG * v); };
    if (nv > 0) {
        dma_a(0, 0);
        stage(0, 0);
        stage(1, 1);
    }

    // LoRA slab(s): acc = scale * B[p rows] . T[m rows]^T, before the weight product.
    const LoraDev &lo = a.lora[seg];
    if (!PAIR && lo.has && split == 0 && g == 0) {
        const int r = lane & 31, kh = (lane >> 5) * 8;
        for (int k0 = 0; k0 < lo.rank; k0 += 16) {
            const int lim = lo.rank - (k0 + kh);
            u32x4_t fa[TP], fb[TM];
#pragma unroll
            for (int i = 0; i < TP; ++i) {
                const int64_t p = p0 + wp * (BP / WP) + i * 32 + r;
                fa[i] = (p < w.rows && lim > 0)
                            ? lora_row8(lo.b + p * lo.rank + k0 + kh, lim, lo.vec)
                            : (u32x4_t){0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int64_t m = m0 + wm * (BM / WM) + j * 32 + r;
                fb[j] = (m < a.M && lim > 0)
                            ? lora_row8(lo.t + m * lo.rank + k0 + kh, lim, lo.vec)
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

    if (ci < 256) {
        const float one = ci == 0 ? 1.0f : 0.0f;  // the table of a weight without nested absmax
        s_code2[0][ci] = a.w[seg].nested ? __builtin_bit_cast(float, c2a) : one;
        if constexpr (PAIR) s_code2[1][ci] = a.w[1].nested ? __builtin_bit_cast(float, c2b) : one;
    }
    __syncthreads();  // tables
    uint8_t *sW[2] = {sT[g][0], sT[g][1]};
    uint8_t *sA[2] = {sT[g][0] + BP * ROWB, sT[g][1] + BP * ROWB};
    if (nv > 0) {
        {
            const Nf4Table tb = make_table_half<DT>(hc, absmax_val(w, wt[0].abs, code2));
#pragma unroll
            for (int q = 0; q < 4; ++q) wt[0].store_part(sW[0], tb, hc.selbase, q);
        }
        wait_dma();
        __syncthreads();
        int64_t v = 0;
        for (; v + 1 < nv; v += 2) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const Nf4Table tb = make_table_half<DT>(hc, absmax_val(w, wt[b ^ 1].abs, code2));
                mma_step_interleaved<DT, TP, TM, PH>(
                    acc, sW[b], sA[b], prow0, wm * (BM / WM), [&](int ks) {
                        wt[b ^ 1].store_part(sW[b ^ 1], tb, hc.selbase, ks);
                        if (ks == 0) {
                            dma_a(b ^ 1, v + b + 1);
                            stage(b, v + b + 2);
                        }
                    });
                wait_dma();
                __syncthreads();
            }
        }
        if (v < nv) mma_step<DT, TP, TM, PH>(acc, sW[0], sA[0], prow0, wm * (BM / WM));
    }
    if constexpr (KG > 1) group_sum<TP, TM, KG, NT>(acc, &sT[0][0][0], g);
    if constexpr (PAIR) {
        epilogue_swiglu<DT, TP, TM, EPI == 2, KG>(a, acc, p0 + prow0, a.w[0].rows,
                                                  m0 + wm * (BM / WM), g);
    } else {
        if constexpr (stage_bytes<BP, BM, KG>() >= BM * BP * 2) {
            if (a.vec16_out && bt.nsplit == 1 && !a.bias && !a.accumulate) {
                epilogue_lds<DT, BP, BM, TP, TM, NT, KG>(a, acc, lds, p0, prow0, w.rows,
                                                         a.seg_off[seg], m0, wm * (BM / WM), g);
                return;
            }
        }
        if constexpr (BP == 128 && stage_bytes<BP, BM, KG>() >= BM * BP * 4) {
            if (a.vec16_out && bt.nsplit == 1) {
                epilogue_lds32<DT, BP, BM, TP, TM, NT, KG>(a, acc, lds, p0, prow0, w.rows,
                                                           a.seg_off[seg], m0, wm * (BM / WM), g);
                return;
            }
        }
        if constexpr (BP == 256 && KG == 1 && stage_bytes<BP, BM, KG>() >= BM * 512) {
            if (bt.nsplit > 1 && a.tail_cols % 4 == 0 && (a.seg_off[seg] - a.tail_col0) % 4 == 0) {
                partial_lds<BM, WM, TP, TM, NT>(a, acc, lds, p0, prow0, w.rows, a.seg_off[seg], m0,
                                            wm * (BM / WM), split);
                return;
            }
        }
        epilogue<DT, TP, TM, KG>(a, acc, p0 + prow0, w.rows, a.seg_off[seg], m0 + wm * (BM / WM),
                                 split, bt.nsplit > 1, g);
    }
}

// Row-owning main loop of a 256x256 forward tile: wave w (of 8) owns the 32 weight rows
// p0 + 32 w .. and all 256 activation rows of the tile, and dequantizes its rows straight into
// its MFMA A fragments: the weight tile never goes through LDS and no two waves dequantize the
// same element.  Lane l takes row 32 w + l % 32 and the packed bytes 16 (l / 32) .. + 15 of the
// row's 64-deep step (elements k = 32 (l / 32) + 0 .. 31, one absmax block); its A fragment of
// k-substep ks is dword ks of those bytes (k = 32 (l / 32) + 8 ks + 0 .. 7), and its B
// fragments read the activation chunk 4 (l / 32) + ks of their rows, the same k.  Per step s:
// the table of step s + 1 is built and its A fragments dequantized, a quarter per k-substep,
// among the MFMAs of step s (two A-fragment register sets); the activation tile of step s + 1
// goes to the other LDS stage by LDS DMA and the packed bytes of step s + 2 to the free
// register stage; one barrier.
template <int DT>
__device__ __forceinline__ void fwd_body_rw(const GemmArgs &a, const TileMap &tm, uint32_t blk,
                                            uint8_t *lds, float (*s_code2)[256]) {
    constexpr int BP = 256, BM = 256, NT = 512, TP = 1, TM = 8, NS = 2;
    constexpr int STG = BM * ROWB;  // bytes of one activation stage
    const BlockTile bt = block_tile(a, blk);
    const int split = bt.split;
    const int64_t tile = bt.tile;
    const int seg = seg_of_tile(a, tm, tile);
    const uint32_t local = static_cast<uint32_t>(tile - tm.tile_start[seg]);
    const uint32_t mtl = static_cast<uint32_t>(tm.m_tiles);
    const int64_t p0 = uniform64(tm.row0[seg] + static_cast<int64_t>(local / mtl) * BP);
    const int64_t m0 = uniform64(static_cast<int64_t>(local % mtl) * BM);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const DevWeight w = a.w[seg];
    const int64_t K = a.K;
    const int64_t steps = K / BR;
    const int64_t per = bt.nsplit > 1 ? a.per_split : steps;
    const int64_t s0 = uniform64(split * per);
    const int64_t s1 = uniform64(s0 + per < steps ? s0 + per : steps);
    const int64_t nv = s1 - s0;

    const int ci = static_cast<int>(threadIdx.x);
    const uint32_t c2a = bload4(make_rsrc(a.w[seg].code2, a.w[seg].nested ? 1024 : 0), ci * 4);
    const float *code2 = s_code2[0];
    float code_r[16];
    load_code_sgpr(w.code, code_r);
    const int lane = threadIdx.x & 63;
    const int r32 = lane & 31, kh = lane >> 5;
    const int prow0 = wave * 32;

    float16_t acc[TP][TM];
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[0][j] = (float16_t){};

    // this lane's 16 packed bytes and absmax block of step 0 (rows past the weight read zero)
    const WeightRsrc wr = weight_rsrc(w);
    const int64_t wrow = p0 + prow0 + r32;
    const int wpk = static_cast<int>(wrow * (K >> 1) + kh * 16);
    const int wblk = static_cast<int>(wrow * (K >> wr.bs_shift));
    struct Raw {
        u32x4_t raw;
        AbsIn abs;
    };
    auto wload = [&](Raw &r, int64_t u) {
        const int st = static_cast<int>(s0 + u);
        r.raw = bload16(wr.packed, wpk + st * (BR / 2));
        r.abs = absmax_bload(wr, wblk + ((st * BR) >> wr.bs_shift));
    };
    const rsrc_t ar = act_rsrc<BM>(a, m0);
    // activation DMA: wave w sends rows 32 w .. 32 w + 31 (4 blocks of 8 rows), lane i writing
    // position i & 7 of row i >> 3 of a block (swz layout)
    int adoff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = (wave * 4 + j) * 8 + (lane >> 3);
        adoff[j] = row * static_cast<int>(a.ld_act) * 2 + (((lane & 7) ^ ((row >> 1) & 7)) << 4);
    }
    const uint32_t lds_a =
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t *)lds)) +
        wave * 32 * ROWB;
    auto dma_a = [&](int b, int64_t u) {
        const int kb = static_cast<int>(s0 + u) * (BR * 2);
        const uint32_t base = __builtin_amdgcn_readfirstlane(lds_a + b * STG);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                         :
                         : "s"(base + j * 8 * ROWB), "v"(adoff[j]), "s"(ar), "s"(kb)
                         : "memory", "m0");
        }
    };
    // Every DMA is followed by exactly one register stage's 3 loads before this wait.
    auto wait_dma = [] { asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); };

    Raw rs[2] = {};
    if (nv > 0) {
        dma_a(0, 0);
        wload(rs[0], 0);
        wload(rs[1], 1);
    }

    const LoraDev &lo = a.lora[seg];
    if (lo.has && split == 0) {
        const int kq = kh * 8;
        for (int k0 = 0; k0 < lo.rank; k0 += 16) {
            const int lim = lo.rank - (k0 + kq);
            u32x4_t fa, fb[TM];
            {
                const int64_t p = p0 + prow0 + r32;
                fa = (p < w.rows && lim > 0) ? lora_row8(lo.b + p * lo.rank + k0 + kq, lim, lo.vec)
                                             : (u32x4_t){0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int64_t m = m0 + j * 32 + r32;
                fb[j] = (m < a.M && lim > 0) ? lora_row8(lo.t + m * lo.rank + k0 + kq, lim, lo.vec)
                                             : (u32x4_t){0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int j = 0; j < TM; ++j) acc[0][j] = mfma32<DT>(fa, fb[j], acc[0][j]);
        }
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[0][j] *= lo.scale;
    }

    if (ci < 256) s_code2[0][ci] = a.w[seg].nested ? __builtin_bit_cast(float, c2a) : (ci == 0 ? 1.0f : 0.0f);
    __syncthreads();  // tables

    auto dword = [](const u32x4_t &v, int q) { return q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w; };
    // B fragment of k-substep ks, m fragment j, from activation stage b
    auto bfrag = [&](int b, int ks, int j) {
        return *reinterpret_cast<const u32x4_t *>(lds + b * STG + swz(j * 32 + r32, kh * 4 + ks));
    };
    // A fragments: fa[ks] holds k-substep ks of the current step until that substep's MFMAs are
    // issued, then the next step's (one register set)
    u32x4_t fa[4];
    if (nv > 0) {
        const Nf4Table tb = make_table<DT>(code_r, absmax_val(w, rs[0].abs, code2));
#pragma unroll
        for (int q = 0; q < 4; ++q) fa[q] = lookup8(tb, dword(rs[0].raw, q));
        wload(rs[0], 2);
        wait_dma();
        __syncthreads();
        // Step v from LDS stage B = v & 1 (B a constant: the loop runs two steps per pass); the
        // next step's fragments from register stage B ^ 1 (step v + 1), whose loads of step v + 3
        // follow its last use; the DMA of step v + 1 into stage B ^ 1 after the first k-substep.
        int64_t v = 0;
        auto body = [&](auto bc) {
            constexpr int B = decltype(bc)::value;
            const Nf4Table tb = make_table<DT>(code_r, absmax_val(w, rs[B ^ 1].abs, code2));
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                u32x4_t fb[TM];
#pragma unroll
                for (int j = 0; j < TM; ++j) fb[j] = bfrag(B, ks, j);
#pragma unroll
                for (int j = 0; j < TM; ++j) acc[0][j] = mfma32<DT>(fa[ks], fb[j], acc[0][j]);
                fa[ks] = lookup8(tb, dword(rs[B ^ 1].raw, ks));
                if (ks == 0) dma_a(B ^ 1, v + B + 1);
                if (ks == 3) wload(rs[B ^ 1], v + B + 3);
                __builtin_amdgcn_sched_barrier(0);  // one k-substep's work at a time
            }
            wait_dma();
            __syncthreads();
        };
        for (; v + 1 < nv; v += 2) {
            body(std::integral_constant<int, 0>{});
            body(std::integral_constant<int, 1>{});
        }
        if (v < nv) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                u32x4_t fb[TM];
#pragma unroll
                for (int j = 0; j < TM; ++j) fb[j] = bfrag(0, ks, j);
#pragma unroll
                for (int j = 0; j < TM; ++j) acc[0][j] = mfma32<DT>(fa[ks], fb[j], acc[0][j]);
            }
        }
    }
    if (a.vec16_out && bt.nsplit == 1 && !a.bias && !a.accumulate) {
        epilogue_lds<DT, BP, BM, TP, TM, NT>(a, acc, lds, p0, prow0, w.rows, a.seg_off[seg], m0, 0);
        return;
    }
    if (bt.nsplit > 1 && a.tail_cols % 4 == 0 && (a.seg_off[seg] - a.tail_col0) % 4 == 0) {
        partial_lds<BM, 1, TP, TM, NT>(a, acc, lds, p0, prow0, w.rows, a.seg_off[seg], m0, 0, split);
        return;
    }
    epilogue<DT, TP, TM>(a, acc, p0 + prow0, w.rows, a.seg_off[seg], m0, split, bt.nsplit > 1);
}

template <int DT>
__global__ __launch_bounds__(512) void fwd_rw_kernel(const GemmArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[stage_bytes<256, 256, 1>()];
    __shared__ float s_code2[1][256];
    fwd_body_rw<DT>(a, a.map[0], blockIdx.x, lds, s_code2);
}


template <int DT, int BP, int BM, int WP, int WM, int EPI = 0, int KG = 1>
__global__ __launch_bounds__(KG *WP *WM * 64) void fwd_kernel(const GemmArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[stage_bytes<BP, BM, KG>()];
    __shared__ float s_code2[EPI != 0 ? 2 : 1][256];
    fwd_body<DT, BP, BM, WP, WM, EPI, KG>(a, a.map[0], blockIdx.x, lds, s_code2);
}

// A two-part launch: workgroups [0, blocks0) run 256x256 tiles over the first part's map, the
// rest 128x128 tiles with two k-groups over the second part's (both 512 threads, the same
// staging LDS), so that the second part's workgroups start on the CUs the first part frees.
template <int DT, int EPI>
__global__ __launch_bounds__(512) void fwd_head_tail_kernel(const GemmArgs a) {
    static_assert(stage_bytes<256, 256, 1>() == stage_bytes<128, 128, 2>(), "one LDS layout");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[stage_bytes<256, 256, 1>()];
    __shared__ float s_code2[EPI != 0 ? 2 : 1][256];
    const uint32_t b0 = static_cast<uint32_t>(a.blocks0);
    if (blockIdx.x < b0) {
        if constexpr (EPI == 0) fwd_body_rw<DT>(a, a.map[0], blockIdx.x, lds, s_code2);
        else fwd_body<DT, 256, 256, 2, 4, EPI, 1>(a, a.map[0], blockIdx.x, lds, s_code2);
    } else
        fwd_body<DT, 128, 128, 2, 2, EPI, 2>(a, a.map[1], blockIdx.x - b0, lds, s_code2);
}

// ------------------------------------------------------------------------ decode forward path
//
// Y = X W^T for M <= 16 tokens with K a multiple of 128 (decode), bound by the dequant VALU work
// and HBM.  A workgroup owns 16 weight rows of one segment and its NW waves split the
// reduction into contiguous ranges of 128-deep super-steps.  In a super-step lane group
// g = lane / 16 takes k = 32g .. 32g + 31 of its row (16 packed bytes inside one absmax block)
// and k-substep ks the 8 values 32g + 8ks ..; the activation B fragments use the same k order
// (64 contiguous bytes of token lane % 16; lanes of tokens >= M load nothing and keep zeros).
// The packed weights run WS super-steps ahead and the activations XS; prefetches past a
// wave's range are clamped to its last super-step (cached bytes), so the loop has no
// branches.  The waves' 16x16 partial tiles are added in wave order through LDS
// (deterministic); no split-K.
constexpr int64_t kDecodeMaxM = 16;
constexpr int DK = 128;  // decode super-step
constexpr int kDecodeWavesPerSimd = 6;  // at most 80 VGPRs

template <int DT>
__device__ __forceinline__ void epilogue16(const GemmArgs &a, const float4_t &acc, int64_t p,
                                           int64_t p_end, int64_t col_off, int64_t m) {
    if (m >= a.M || p >= p_end) return;
    const int64_t col = col_off + p;
    float v[4] = {acc.x, acc.y, acc.z, acc.w};
    if (a.bias) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (p + q < p_end) v[q] += to_f32<DT>(a.bias[col + q]);
    }
    uint16_t *dst = static_cast<uint16_t *>(a.out) + m * a.ld_out + col;
    if (p + 4 <= p_end && a.vec_out) {
        u32x2_t o;
        o.x = pack2<DT>(v[0], v[1]);
        o.y = pack2<DT>(v[2], v[3]);
        *reinterpret_cast<u32x2_t *>(dst) = o;
    } else {
        for (int q = 0; q < 4; ++q)
            if (p + q < p_end) dst[q] = from_f32<DT>(v[q]);
    }
}

// The fp32 partial sums of a split reduction, lane layout of epilogue16: partials
// [splits][M][n_out] (tail_col0 = 0) for split_reduce_kernel, which adds the bias and rounds.
__device__ __forceinline__ void partial16(const GemmArgs &a, const float4_t &acc, int64_t p,
                                          int64_t p_end, int64_t col_off, int64_t m, int split) {
    if (m >= a.M || p >= p_end) return;
    float *dst = a.partial + (static_cast<int64_t>(split) * a.M + m) * a.tail_cols + col_off + p;
    if (p + 4 <= p_end && ((a.tail_cols | col_off) & 3) == 0) {
        *reinterpret_cast<float4_t *>(dst) = acc;
    } else {
        const float v[4] = {acc.x, acc.y, acc.z, acc.w};
        for (int q = 0; q < 4; ++q)
            if (p + q < p_end) dst[q] = v[q];
    }
}

template <int DT, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(kDecodeWavesPerSimd)))
void decode_kernel(const GemmArgs a) {
    constexpr int WS = 4, XS = 2;
    __shared__ float s_code2[256];
    __shared__ float4_t s_red[NW > 1 ? NW - 1 : 1][64];

    const int64_t tile = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(blockIdx.x));
    const int seg = seg_of_tile(a, a.map[0], tile);
    const int64_t p0 = uniform64((tile - a.map[0].tile_start[seg]) * 16);
    const DevWeight w = a.w[seg];
    const int64_t K = a.K;
    const int ss = static_cast<int>(K / DK);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int per = (ss + NW - 1) / NW;
    const int w0 = wave * per < ss ? wave * per : ss;
    const int w1 = w0 + per < ss ? w0 + per : ss;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;

    for (int i = threadIdx.x; i < 256; i += NW * 64) s_code2[i] = code2_entry(w, i);
    float code_r[16];
    load_code_sgpr(w.code, code_r);

    const WeightRsrc wr = weight_rsrc(w);
    const int64_t row = p0 + r;
    const int wpk = static_cast<int>(row * (K >> 1) + 16 * g);
    const int wblk = static_cast<int>(row * (K >> wr.bs_shift));
    const int64_t mrows = a.M < 16 ? a.M : 16;
    const rsrc_t xr = make_rsrc(a.act, ((mrows - 1) * a.ld_act + a.act_cols) * 2);
    const int xoff = static_cast<int>((r * a.ld_act + 32 * g) * 2);

    struct WStage {
        u32x4_t raw;
        AbsIn abs;
    };
    struct XStage {
        u32x4_t x[4];
    };
    const int last = w1 > w0 ? w1 - 1 : w0;
    auto cl = [&](int v) { return v < last ? v : last; };
    auto wload = [&](WStage &s, int st) {
        s.raw = bload16(wr.packed, wpk + st * (DK / 2));
        s.abs = absmax_bload(wr, wblk + ((st * DK + 32 * g) >> wr.bs_shift));
    };
    // lanes of tokens >= M issue no activation loads (their fragments stay zero): at M = 1 the
    // vector memory unit then spends its address cycles on the weights
    const bool xlane = r < mrows;
    auto xload = [&](XStage &s, int st) {
        if (xlane) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) s.x[ks] = bload16(xr, xoff + st * (DK * 2) + ks * 16);
        }
    };
    // LoRA slab on the last wave, before any prefetch is in flight (its loads are waited for
    // in full): acc = scale * B[p rows] . T[m rows]^T, rank in 32-deep MFMA chunks, zero-padded
    float4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const LoraDev &lo = a.lora[seg];
    if (lo.has && wave == NW - 1) {
        for (int k0 = 0; k0 < lo.rank; k0 += 32) {
            const int lim = lo.rank - (k0 + 8 * g);
            const u32x4_t fa = (row < w.rows && lim > 0) ? gather8(lo.b + row * lo.rank + k0 + 8 * g, 1, lim)
                                                         : (u32x4_t){0u, 0u, 0u, 0u};
            const u32x4_t fb = (r < a.M && lim > 0) ? gather8(lo.t + r * lo.rank + k0 + 8 * g, 1, lim)
                                                    : (u32x4_t){0u, 0u, 0u, 0u};
            acc = mfma16<DT>(fa, fb, acc);
        }
        acc *= lo.scale;
    }

    // Loads complete in issue order, so each super-step issues its activation prefetch before
    // its weight prefetch: waiting for the activations of step s then never waits for weights
    // younger than step s + WS - 1.
    WStage ws[WS];
    XStage xs[XS] = {};
#pragma unroll
    for (int b = 0; b < XS; ++b) xload(xs[b], cl(w0 + b));
#pragma unroll
    for (int b = 0; b < WS; ++b) wload(ws[b], cl(w0 + b));
    __syncthreads();  // code2 table

    auto compute = [&](const WStage &s, const XStage &x) {
        const Nf4Table tb = make_table<DT>(code_r, absmax_val(w, s.abs, s_code2));
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const uint32_t wd = ks == 0 ? s.raw.x : ks == 1 ? s.raw.y : ks == 2 ? s.raw.z : s.raw.w;
            acc = mfma16<DT>(lookup8(tb, wd), x.x[ks], acc);
        }
    };
    int st = w0;
    for (; st + WS <= w1; st += WS) {
#pragma unroll
        for (int b = 0; b < WS; ++b) {
            compute(ws[b], xs[b % XS]);
            __builtin_amdgcn_sched_barrier(0);
            xload(xs[b % XS], cl(st + b + XS));
            wload(ws[b], cl(st + b + WS));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int b = 0; b < WS - 1; ++b) {
        if (st + b < w1) {
            compute(ws[b], xs[b % XS]);
            xload(xs[b % XS], cl(st + b + XS));
        }
    }

    if constexpr (NW > 1) {
        if (wave > 0) s_red[wave - 1][lane] = acc;
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int v = 0; v < NW - 1; ++v) acc += s_red[v][lane];
        }
    }
    if (wave == 0) epilogue16<DT>(a, acc, p0 + 4 * g, w.rows, a.seg_off[seg], r);
}

// ------------------------------------------------------------------ skinny forward path
//
// Y = X W^T for 2 < M <= 64 tokens (decode steps and small batches) with K a multiple of the
// super-step DKS (128 or 256), on v_mfma_f32_16x16x32: A = 16 weight rows dequantized straight
// into registers, B = 16 tokens.  A workgroup of RT x KP waves owns 16 RT weight rows of one
// segment: wave w takes the 16-row tile w % RT and the k-part w / RT (KP contiguous ranges of
// DKS-deep super-steps).  The activations, the one operand all of a workgroup's row tiles
// share, are read from memory once per workgroup into LDS: in round r the stage holds, for each
// k-part kp, its super-step kp * per + r for the 16 MT tokens ([KP][16 MT][DKS k], two stages,
// loaded through registers one round ahead by every thread, token rows >= M reading zero), and
// each wave reads its MT B fragments per k-substep from there.  (One workgroup per 16 rows,
// each reading all of X from L2, moved twice the weight bytes at M = 8.)  Lane l takes row
// 16 rt + l % 16 and the k values DKS / 4 * (l / 16) .. + DKS / 4 - 1 of a super-step (DKS / 8
// packed bytes inside one absmax block: blocks are at least 64 wide, so one table per lane and
// super-step); k-substep ks uses the 8 values from DKS / 4 * (l / 16) + 8 ks, A in nibble-plane
// order (lookup8_planes) and B, the same k of token 16 mt + l % 16, stored in that order in LDS
// (plane_order when staged; rows of 2 DKS bytes, 16-byte chunk c of token t at c ^ (t % 16), so
// the 16 tokens of a fragment read hit 16 distinct bank groups).  A wave past the end of its
// k-part (the last part may be shorter) skips the arithmetic of a round but keeps loading and
// meeting the barriers.  The KP partial tiles are added in k-part order through LDS
// (deterministic).  DKS = 256 halves the tables, the barriers and the rounds of DKS = 128 and
// doubles the weight bytes in flight; its stages need twice the LDS.
constexpr int64_t kSkinnyMaxM = 64;

// Half tables (make_table_half16) at DKS = 128, except where their 8 code registers per lane
// would cost a workgroup per CU (the register counts of the compiled kernels: 1 token group x
// 8 k-parts, 2 x 2 row tiles, 4 x 8 row tiles, and 2 x 8 with the down-projection in the launch).
constexpr bool skinny_half(int mt, int rt, int kp, int dks, bool fx) {
    return dks == 128 && !(mt == 1 && kp == 8 && !fx) && !(mt == 2 && rt == 2 && !fx) &&
           !(mt == 4 && rt == 8) && !(mt == 2 && rt == 8 && fx);
}

template <int DT, int MT, int RT, int KP, int DKS, bool FX>
__global__ __launch_bounds__(RT * KP * 64) void skinny_kernel(const GemmArgs a) {
    constexpr int NW = RT * KP, NT = NW * 64, MP = 16 * MT;
    constexpr int WS = 3;                 // weight register stages
    constexpr int NSUB = DKS / 32;        // k-substeps of a super-step
    constexpr int XROW = DKS * 2;         // LDS bytes of one token's super-step
    constexpr int CPT = DKS / 8;          // its 16-byte chunks
    constexpr int RS = MP + (FX ? 16 : 0);  // stage rows per k-part: tokens, then A's rows
    constexpr int XSTG = KP * RS * XROW;  // one activation stage
    constexpr int XCH = KP * MP * CPT;    // its 16-byte chunks of activations
    constexpr int CH = (XCH + NT - 1) / NT;
    constexpr int ACH = KP * 16 * CPT;    // ... and of A's rows
    constexpr int CHA = FX ? (ACH + NT - 1) / NT : 0;
    static_assert(DKS == 128 || DKS == 256, "super-steps of 128 or 256");
    static_assert(2 * XSTG + 1024 + (FX ? MP * 32 : 0) <= 160 * 1024, "two stages fit in LDS");
    static_assert(((KP - 1) * RT * MT + (FX ? (KP - 1) * MT : 0)) * 64 * 16 <= 2 * XSTG,
                  "the k-part sums fit in the stages");
    __shared__ __attribute__((aligned(16))) uint8_t s_x[2 * XSTG];
    __shared__ float s_code2[256];
    __shared__ __attribute__((aligned(16))) uint16_t s_t[FX ? MP : 1][16];  // T, token-major

    // workgroup b: row tile b / splits, reduction split b % splits (super-steps
    // [split * per_split, + per_split) of K)
    const int nsplit = a.splits;
    const int bid = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x));
    const int64_t tile = bid / nsplit;
    const int split = bid - static_cast<int>(tile) * nsplit;
    const int seg = seg_of_tile(a, a.map[0], tile);
    const int64_t p0 = uniform64((tile - a.map[0].tile_start[seg]) * (16 * RT));
    const DevWeight w = a.w[seg];
    const int64_t K = a.K;
    const int ss = static_cast<int>(K / DKS);
    const int s0 = split * static_cast<int>(a.per_split);
    const int s1 = s0 + static_cast<int>(a.per_split) < ss ? s0 + static_cast<int>(a.per_split) : ss;
    const int per = (s1 - s0 + KP - 1) / KP;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int rt = wave % RT, kp = wave / RT;
    const int my0 = s0 + kp * per;
    const int my_n = s1 - my0 < per ? (s1 - my0 > 0 ? s1 - my0 : 0) : per;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;
    const LoraDev &lo = a.lora[seg];
    // the LoRA down-projection T = X A^T of this segment, computed here: A's rows ride in the
    // activation stages and the first row tile's waves add its products (one per k-substep)
    const bool fx = FX && lo.xa != nullptr;
    const bool fx_wave = fx && rt == 0;

    for (int i = threadIdx.x; i < 256; i += NT) s_code2[i] = code2_entry(w, i);
    float code_r[16];
    load_code_sgpr(w.code, code_r);
    // lane groups g and g ^ 1 cover one absmax block at DKS = 128 (skinny_half below)
    const Nf4HalfCodes hc = half_codes16(code_r);

    // weights: DKS / 8 packed bytes of this lane's row per super-step; a wave's loads past its
    // part repeat its last super-step (cached bytes, never used)
    const WeightRsrc wr = weight_rsrc(w);
    const int64_t row = p0 + 16 * rt + r;
    const int wpk = static_cast<int>(row * (K >> 1) + (DKS / 8) * g);
    const int wblk = static_cast<int>(row * (K >> wr.bs_shift));
    const int last = my_n > 0 ? my0 + my_n - 1 : 0;
    struct WStage {
        u32x4_t raw[NSUB / 4];
        AbsIn abs;
    };
    auto wload = [&](WStage &s, int v) {
        const int st = my0 + v < last ? my0 + v : last;
#pragma unroll
        for (int q = 0; q < NSUB / 4; ++q) s.raw[q] = bload16(wr.packed, wpk + st * (DKS / 2) + 16 * q);
        s.abs = absmax_bload(wr, wblk + ((st * DKS + (DKS / 4) * g) >> wr.bs_shift));
    };
    // activations: chunk c of a stage is k-part c / (CPT MP), token (c / CPT) % MP, 16-byte
    // column c % CPT; super-steps past K read the next row's bytes or zero (never used)
    const int64_t mrows = a.M < MP ? a.M : MP;
    const rsrc_t xr = make_rsrc(a.act, ((mrows - 1) * a.ld_act + a.act_cols) * 2);
    const int ldb = static_cast<int>(a.ld_act) * 2;
    u32x4_t xs[CH];
    u32x4_t xsa[CHA > 0 ? CHA : 1];
    // A's rows (rank <= 16; rows past the rank read zero)
    const rsrc_t ar = make_rsrc(lo.xa, fx ? int64_t(lo.rank) * K * 2 : 0);
    auto xload = [&](int rd) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = static_cast<int>(threadIdx.x) + i * NT;
            if (XCH % NT != 0 && c >= XCH) continue;
            const int kq = c / (MP * CPT), t = (c / CPT) % MP, kc = c % CPT;
            xs[i] = bload16(xr, t * ldb + (s0 + kq * per + rd) * XROW + kc * 16);
        }
        if (fx) {
#pragma unroll
            for (int i = 0; i < CHA; ++i) {
                const int c = static_cast<int>(threadIdx.x) + i * NT;
                if (ACH % NT != 0 && c >= ACH) continue;
                const int kq = c / (16 * CPT), j = (c / CPT) % 16, kc = c % CPT;
                xsa[i] = bload16(ar, j * static_cast<int>(K * 2) + (s0 + kq * per + rd) * XROW + kc * 16);
            }
        }
    };
    auto xstore = [&](int b) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = static_cast<int>(threadIdx.x) + i * NT;
            if (XCH % NT != 0 && c >= XCH) continue;
            const int kq = c / (MP * CPT), t = (c / CPT) % MP, kc = c % CPT;
            *reinterpret_cast<u32x4_t *>(s_x + b * XSTG + (kq * RS + t) * XROW +
                                         ((kc ^ (t & 15)) << 4)) = plane_order(xs[i]);
        }
        if (fx) {
#pragma unroll
            for (int i = 0; i < CHA; ++i) {
                const int c = static_cast<int>(threadIdx.x) + i * NT;
                if (ACH % NT != 0 && c >= ACH) continue;
                const int kq = c / (16 * CPT), j = (c / CPT) % 16, kc = c % CPT;
                *reinterpret_cast<u32x4_t *>(s_x + b * XSTG + (kq * RS + MP + j) * XROW +
                                             ((kc ^ j) << 4)) = plane_order(xsa[i]);
            }
        }
    };

    float4_t acc[MT], acc_t[FX ? MT : 1];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mt = 0; mt < (FX ? MT : 1); ++mt) acc_t[mt] = (float4_t){0.f, 0.f, 0.f, 0.f};
    if (lo.has && !fx && kp == 0 && split == 0) {
        for (int k0 = 0; k0 < lo.rank; k0 += 32) {
            const int lim = lo.rank - (k0 + 8 * g);
            const u32x4_t fa = (row < w.rows && lim > 0) ? gather8(lo.b + row * lo.rank + k0 + 8 * g, 1, lim)
                                                         : (u32x4_t){0u, 0u, 0u, 0u};
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int64_t m = 16 * mt + r;
                const u32x4_t fb = (m < a.M && lim > 0) ? gather8(lo.t + m * lo.rank + k0 + 8 * g, 1, lim)
                                                        : (u32x4_t){0u, 0u, 0u, 0u};
                acc[mt] = mfma16<DT>(fa, fb, acc[mt]);
            }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] *= lo.scale;
    }

    WStage wst[WS];
#pragma unroll
    for (int b = 0; b < WS; ++b) wload(wst[b], b);
    xload(0);
    xstore(0);
    __syncthreads();  // code2 table, activation stage 0

    auto compute = [&](const WStage &s, int b) {
        // DKS = 128: the lane groups g and g ^ 1 cover the two halves of one absmax block and
        // build its table together (make_table_half16)
        constexpr bool HALF = skinny_half(MT, RT, KP, DKS, FX);
        const Nf4Table tb = HALF ? make_table_half16<DT>(hc, absmax_val(w, s.abs, s_code2))
                                 : make_table<DT>(code_r, absmax_val(w, s.abs, s_code2));
        const uint8_t *xb = s_x + b * XSTG + kp * RS * XROW;
#pragma unroll
        for (int ks = 0; ks < NSUB; ++ks) {
            const u32x4_t &raw = s.raw[ks / 4];
            const uint32_t wd = ks % 4 == 0 ? raw.x : ks % 4 == 1 ? raw.y : ks % 4 == 2 ? raw.z : raw.w;
            const u32x4_t fa = HALF ? lookup8_planes_s(tb, wd, hc.selbase) : lookup8_planes(tb, wd);
            u32x4_t fa_t = (u32x4_t){0u, 0u, 0u, 0u};
            if (FX && fx_wave)
                fa_t = *reinterpret_cast<const u32x4_t *>(xb + (MP + r) * XROW + (((NSUB * g + ks) ^ r) << 4));
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int t = 16 * mt + r;
                const u32x4_t fb = *reinterpret_cast<const u32x4_t *>(
                    xb + t * XROW + (((NSUB * g + ks) ^ (t & 15)) << 4));
                acc[mt] = mfma16<DT>(fa, fb, acc[mt]);
                if (FX && fx_wave) acc_t[mt] = mfma16<DT>(fa_t, fb, acc_t[mt]);
            }
        }
    };
    // round rd: activations in stage rd & 1 (landed before the previous barrier); the next
    // round's go to registers first and to the other stage after this round's arithmetic
    auto round = [&](WStage &s, int rd) {
        if (rd + 1 < per) xload(rd + 1);
        if (rd < my_n) compute(s, rd & 1);
        wload(s, rd + WS);
        if (rd + 1 < per) xstore((rd + 1) & 1);
        __syncthreads();
    };
    int rd = 0;
    for (; rd + WS <= per; rd += WS) {
#pragma unroll
        for (int b = 0; b < WS; ++b) round(wst[b], rd + b);
    }
#pragma unroll
    for (int b = 0; b < WS - 1; ++b)
        if (rd + b < per) round(wst[b], rd + b);

    if constexpr (KP > 1) {
        float4_t *red = reinterpret_cast<float4_t *>(s_x);  // the stages are free now
        float4_t *red_t = red + (KP - 1) * RT * MT * 64;
        if (kp > 0) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) red[(((kp - 1) * RT + rt) * MT + mt) * 64 + lane] = acc[mt];
            if (FX && fx_wave) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) red_t[((kp - 1) * MT + mt) * 64 + lane] = acc_t[mt];
            }
        }
        __syncthreads();
        if (kp == 0) {
#pragma unroll
            for (int q = 1; q < KP; ++q)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) acc[mt] += red[(((q - 1) * RT + rt) * MT + mt) * 64 + lane];
            if (FX && fx_wave) {
#pragma unroll
                for (int q = 1; q < KP; ++q)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc_t[mt] += red_t[((q - 1) * MT + mt) * 64 + lane];
            }
        }
    }
    if constexpr (FX) {
        if (fx) {
            // T rounded to the GEMM dtype (as the standalone down-projection writes it): ranks
            // 4 g .. 4 g + 3 of token 16 mt + r in this lane; into LDS for the slab below, and
            // out to t_out by the segment's first workgroup (the backward pass needs T)
            if (fx_wave && kp == 0) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int t = 16 * mt + r;
                    u32x2_t v;
                    v.x = pack2<DT>(acc_t[mt].x, acc_t[mt].y);
                    v.y = pack2<DT>(acc_t[mt].z, acc_t[mt].w);
                    *reinterpret_cast<u32x2_t *>(&s_t[t][4 * g]) = v;
                    if (p0 == 0 && t < a.M) {
                        const uint16_t h[4] = {static_cast<uint16_t>(v.x), static_cast<uint16_t>(v.x >> 16),
                                               static_cast<uint16_t>(v.y), static_cast<uint16_t>(v.y >> 16)};
                        for (int q = 0; q < 4; ++q)
                            if (4 * g + q < lo.rank) lo.t_out[t * lo.rank + 4 * g + q] = h[q];
                    }
                }
            }
            __syncthreads();
            // the slab: Y_seg += scale * T B^T, k over the 16 (zero-padded) ranks
            if (kp == 0) {
                const int lim = lo.rank - 8 * g;
                const u32x4_t fa = (row < w.rows && lim > 0) ? gather8(lo.b + row * lo.rank + 8 * g, 1, lim)
                                                             : (u32x4_t){0u, 0u, 0u, 0u};
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const u32x4_t fb = g < 2 ? *reinterpret_cast<const u32x4_t *>(&s_t[16 * mt + r][8 * g])
                                             : (u32x4_t){0u, 0u, 0u, 0u};
                    acc[mt] += mfma16<DT>(fa, fb, (float4_t){0.f, 0.f, 0.f, 0.f}) * lo.scale;
                }
            }
        }
    }
    if (kp == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            if (nsplit > 1)
                partial16(a, acc[mt], p0 + 16 * rt + 4 * g, w.rows, a.seg_off[seg], 16 * mt + r, split);
            else
                epilogue16<DT>(a, acc[mt], p0 + 16 * rt + 4 * g, w.rows, a.seg_off[seg], 16 * mt + r);
        }
    }
}

// ------------------------------------------------------------------- small-M forward path
//
// Y = X W^T for M <= 32 * MT tokens (the decode regime; the planner launches MT = 1 only, the
// tiled GEMMs being faster from 33 tokens on), bound by reading the packed weights.  A workgroup owns 32 weight rows of one segment; its NW waves split the reduction,
// each dequantizing its rows straight into MFMA A-fragment registers (no LDS staging) and
// reading its activation B-fragments from global memory (rows >= M read as zero from the
// buffer range check).  Inside a 64-deep step both operands use the same k order: lane half h
// takes k = 32h .. 32h+31 and k-substep ks the 8 values 32h + 8ks .. 32h + 8ks + 7, so each lane
// loads its row's 16 packed bytes and its activation row's 64 bytes contiguously.  The NW
// partial tiles are added through LDS in wave order (deterministic) and leave through the GEMM
// epilogue.  At most 128 VGPRs for one activation fragment (four waves per SIMD keep enough
// loads in flight), 256 for two.
template <int DT, int MT, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(MT == 1 ? 4 : 2)))
void gemv_kernel(const GemmArgs a) {
    __shared__ float s_code2[256];
    __shared__ float4_t s_red[NW / 2][MT * 4][64];

    const BlockTile bt = block_tile(a, blockIdx.x);
    const int split = bt.split;
    const int64_t tile = bt.tile;
    const int seg = seg_of_tile(a, a.map[0], tile);
    const int64_t p0 = (tile - a.map[0].tile_start[seg]) * 32;
    const DevWeight w = a.w[seg];
    const int64_t K = a.K;
    const int64_t steps = K / BR;
    const int64_t per = bt.nsplit > 1 ? a.per_split : steps;
    const int64_t s0 = split * per;
    const int64_t s1 = s0 + per < steps ? s0 + per : steps;
    // wave-uniform: the step range below lives in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int64_t pw = (s1 - s0 + NW - 1) / NW;
    const int64_t w0 = s0 + wave * pw;
    const int64_t w1 = w0 + pw < s1 ? w0 + pw : s1;

    const WeightRsrc wr = weight_rsrc(w);
    const int r = lane & 31, h = lane >> 5;
    const int64_t row = p0 + r;
    const int wpk = static_cast<int>(row * (K >> 1) + 16 * h);
    const int wblk = static_cast<int>(row * (K >> wr.bs_shift));
    const int64_t mrows = a.M < 32 * MT ? a.M : 32 * MT;
    const rsrc_t xr = make_rsrc(a.act, ((mrows - 1) * a.ld_act + a.act_cols) * 2);
    int xoff[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) xoff[j] = static_cast<int>(((j * 32 + r) * a.ld_act + 32 * h) * 2);

    // Three register stages of (weights, activations), loaded three steps ahead and issued
    // before anything else, so their latency overlaps the table loads.  Prefetch steps are
    // clamped to the wave's last step, so they re-read cached bytes instead of fetching other
    // waves' rows; the loop body has no branches.
    struct Stage {
        u32x4_t raw;
        AbsIn abs;
        u32x4_t x[MT][4];
    };
    auto load = [&](Stage &g, int64_t st) {
        g.raw = bload16(wr.packed, wpk + static_cast<int>(st) * (BR / 2));
        g.abs = absmax_bload(wr, wblk + static_cast<int>((st * BR) >> wr.bs_shift));
#pragma unroll
        for (int j = 0; j < MT; ++j)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                g.x[j][ks] = bload16(xr, xoff[j] + static_cast<int>(st) * (BR * 2) + ks * 16);
    };
    // table loads first: waiting for them (in issue order) then never waits for the prefetch
    float c2 = 0.f;
    if (threadIdx.x < 256) c2 = code2_entry(w, threadIdx.x);
    float code_r[16];
    load_code_sgpr(w.code, code_r);
    const int64_t last = w1 > w0 ? w1 - 1 : w0;
    auto cl = [&](int64_t v) { return v < last ? v : last; };
    Stage g[3];
#pragma unroll
    for (int b = 0; b < 3; ++b) load(g[b], cl(w0 + b));
    if (threadIdx.x < 256) s_code2[threadIdx.x] = c2;

    float16_t acc[1][MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[0][j] = (float16_t){};
    __syncthreads();  // tables

    // LoRA slab on the last wave (the one with the fewest steps) of split 0:
    // acc = scale * B[p rows] . T[m rows]^T, before its share of the weight product
    const LoraDev &lo = a.lora[seg];
    if (lo.has && split == 0 && wave == NW - 1) {
        const int kh = h * 8;
        for (int k0 = 0; k0 < lo.rank; k0 += 16) {
            const int lim = lo.rank - (k0 + kh);
            const u32x4_t fa = (row < w.rows && lim > 0) ? gather8(lo.b + row * lo.rank + k0 + kh, 1, lim)
                                                         : (u32x4_t){0u, 0u, 0u, 0u};
#pragma unroll
            for (int j = 0; j < MT; ++j) {
                const int64_t m = j * 32 + r;
                const u32x4_t fb = (m < a.M && lim > 0) ? gather8(lo.t + m * lo.rank + k0 + kh, 1, lim)
                                                        : (u32x4_t){0u, 0u, 0u, 0u};
                acc[0][j] = mfma32<DT>(fa, fb, acc[0][j]);
            }
        }
#pragma unroll
        for (int j = 0; j < MT; ++j) acc[0][j] *= lo.scale;
    }

    auto compute = [&](const Stage &g) {
        const Nf4Table tb = make_table<DT>(code_r, absmax_val(w, g.abs, s_code2));
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const uint32_t wd = ks == 0 ? g.raw.x : ks == 1 ? g.raw.y : ks == 2 ? g.raw.z : g.raw.w;
            const u32x4_t fa = lookup8(tb, wd);
#pragma unroll
            for (int j = 0; j < MT; ++j) acc[0][j] = mfma32<DT>(fa, g.x[j][ks], acc[0][j]);
        }
    };
    if (w0 < w1) {
        int64_t st = w0;
        for (; st + 3 <= w1; st += 3) {
#pragma unroll
            for (int b = 0; b < 3; ++b) {
                compute(g[b]);
                load(g[b], cl(st + b + 3));
            }
        }
#pragma unroll
        for (int b = 0; b < 2; ++b)
            if (st + b < w1) compute(g[b]);
    }

    // fixed-order tree reduction of the waves' tiles through LDS (wave v += wave v + half,
    // halving), then wave 0's epilogue
#pragma unroll
    for (int half = NW / 2; half >= 1; half /= 2) {
        if (wave >= half && wave < 2 * half) {
#pragma unroll
            for (int j = 0; j < MT; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    s_red[wave - half][j * 4 + q][lane] =
                        (float4_t){acc[0][j][4 * q], acc[0][j][4 * q + 1], acc[0][j][4 * q + 2],
                                   acc[0][j][4 * q + 3]};
        }
        __syncthreads();
        if (wave < half) {
#pragma unroll
            for (int j = 0; j < MT; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4_t t = s_red[wave][j * 4 + q][lane];
                    acc[0][j][4 * q] += t.x;
                    acc[0][j][4 * q + 1] += t.y;
                    acc[0][j][4 * q + 2] += t.z;
                    acc[0][j][4 * q + 3] += t.w;
                }
        }
        if (half > 1) __syncthreads();
    }
    if (wave == 0) {
        epilogue<DT, 1, MT>(a, acc, p0, w.rows, a.seg_off[seg], 0, split, bt.nsplit > 1);
    }
}

// ---------------------------------------------------------- row-streaming decode path
//
// Y = X W^T for M <= 2 tokens: bound by reading the packed weight once.  A row is cut into 1 KB
// slots of packed bytes (2048 k; lane l of a wave takes the 16 bytes at 16 l, 32 elements inside
// one absmax block) and the slots into K parts of SP <= 2 slots.  A row group owns up to
// kRowsMaxRows rows of one segment, interleaved over the segment's groups (group g takes rows
// g, g + G, g + 2G, .. of the segment's G groups, so that at any time the launch reads one
// contiguous stretch of the weight: measured 2 % faster than consecutive rows per group); a
// wave owns one K part of its group's rows and keeps the part's activations (64 bytes per lane,
// slot and token) in registers for all of them, so the main loop streams weight bytes only.
// An LDS table maps a packed byte to its two codes rounded to the GEMM dtype as one pair
// (code[high nibble] in the low half: element order): a packed byte is one table read and, per
// token, one v_dot2 with the activation pair, accumulated in fp32, and a lane's 32 products are
// then scaled by their block's fp32 absmax (rebuilt as in the other kernels).  The numerics are
// those of bitsandbytes' decode GEMV (no fp16 weight is formed) except that the 16 codes are
// rounded to the GEMM dtype: each product is round16(code[nib]) * x exactly and a block's sum is
// scaled by its absmax in fp32.
//
// The table: with one slot per part (K <= 2048) one 1 KB copy; random bytes make its reads
// ~4-way bank conflicted (the LDS is busy ~5 cycles per read), which the short launches of
// such rows do not feel.  With two slots per part, 64 copies, entry e of copy l at dword
// 64 e + l, so that lane l reads only bank l (no conflicts; the byte address 256 e + 4 l is one
// v_perm of the packed dword and 4 l) and 16-wave workgroups (one per CU) to amortize its 64 KB
// fill: the 7B gate|up and down projections at M = 1 measured 15-18 % faster with it, the
// one-slot 1.5B launches up to 40 % slower (the fill does not pay for itself there).
//
// After each row the lane partials are reduced across the wave in a fixed order (DPP within
// rows of 16 lanes, then the four rows) and lane r keeps the sum of the wave's row r.  Rows with
// several K parts (K > SP x 2048) are shared by the waves of one workgroup, which add their
// parts through LDS in part order after the loop: deterministic.  The LoRA term of a row (lanes
// < rank; the B row is loaded with the row's weight bytes) joins the first part's partial before
// the reduction, the bias is added at the store.  Lanes past a row's end, and slots of a part
// past it, multiply activations that read as zero (their resource ends with the activation
// row), so the loop has no masks; the weight bytes they read belong to the next row or read as
// zero past the weight.  Each wave keeps kRowsRing rows of loads in flight (measured: deeper
// rings were slower), re-reading its last row past its range rather than branching.
constexpr int64_t kRowsMaxM = 2;
constexpr int kRowsMaxParts = 8;    // K <= 8 x 2 x 2048
constexpr int kRowsMaxRows = 64;    // rows per wave: one result lane each
constexpr int kRowsMaxWaves = 16;
constexpr int kRowsRing = 2;        // rows of loads in flight per wave

// The map `a.map[0]`: tile_start[s] = first row group of segment s (cumulative, each segment's
// groups padded to a multiple of a.rows_groups); a workgroup runs a.rows_groups groups x
// a.rows_parts K parts, wave w taking part w % rows_parts of group w / rows_parts.
// (4 waves per SIMD are enough: squeezed for more, the compiler reuses registers that loads
// in flight still target, which waits for them.)
template <int DT, int MT, int SP>
__global__ __launch_bounds__(kRowsMaxWaves * 64) __attribute__((amdgpu_waves_per_eu(4, 4)))
void gemv_rows_kernel(const GemmArgs a) {
    constexpr int RD = kRowsRing;
    constexpr bool kPrivate = SP == 2;  // one table copy per lane (bank)
    __shared__ __attribute__((aligned(1024))) uint32_t s_pair[kPrivate ? 256 * 64 : 256];
    __shared__ float s_code2[256];
    __shared__ float s_part[kRowsMaxWaves][MT][64];
    const int np = a.rows_parts;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int part = wave % np;
    // The workgroup's groups lie in one segment (each segment's groups are padded to whole
    // workgroups), so its table sits at a fixed LDS address and a lookup's address is the
    // packed byte times 4 (one shift with a byte select).
    const TileMap &tm = a.map[0];
    const int64_t grp0 = static_cast<int64_t>(blockIdx.x) * a.rows_groups;
    const int seg = seg_of_tile(a, tm, grp0);
    const int64_t grp = grp0 + wave / np;
    const DevWeight w = a.w[seg];
    const int gs = static_cast<int>(uniform64(tm.tile_start[seg + 1] - tm.tile_start[seg]));
    const int gi = static_cast<int>(uniform64(grp - tm.tile_start[seg]));
    // rows gi, gi + gs, .. (none in a padding group, which loads row 0)
    const int nrows = gi < w.rows ? static_cast<int>((w.rows - gi + gs - 1) / gs) : 0;
    const int64_t lrow0 = nrows > 0 ? gi : 0;
    const int64_t K = a.K;
    const int khalf = static_cast<int>(K / 2);
    const int lane = threadIdx.x & 63;
    const int slot0 = part * SP;
    const WeightRsrc wr = weight_rsrc(w);
    const LoraDev lo = a.lora[seg];
    const bool lora = lo.has && part == 0;
    const float lscale = lora ? lo.scale : 0.0f;
    // Byte and 16-bit operands are loaded as the aligned dwords that hold them and picked out at
    // use: a loop-carried sub-dword load gets a zero-extension at the loop's back edge, which
    // waits for it.  The dword of the last byte may extend past the operand (the host checks
    // that both bases are 4-byte aligned, so it never crosses a page).
    const rsrc_t br = make_rsrc(lo.b, lora ? (w.rows * lo.rank * 2 + 3) & ~int64_t(3) : 0);
    const int64_t nblk = (w.rows * w.cols + w.blocksize - 1) >> w.bs_shift;
    const rsrc_t qr = make_rsrc(w.absmax, w.nested ? (nblk + 3) & ~int64_t(3) : 0);
    const int kb = static_cast<int>(K >> w.bs_shift);  // absmax blocks per row

    // The tables of the workgroup's segment: thread i < 256 (every workgroup has at least 512
    // threads) writes code2 entry i and pair entry i (one copy), or threads 2e and 2e + 1 the
    // 64 copies of pair entry e, before the barrier below.  Their loads go first, from every
    // thread (a branch here would leave them in flight behind the ring loads on some paths,
    // which makes the loop's wait counts conservative).
    const int i = threadIdx.x & 255;
    const int e = kPrivate ? (threadIdx.x >> 1) & 255 : i;
    uint32_t hi, lo2, c2;
    {
        const rsrc_t cr = make_rsrc(w.code, 64);
        const rsrc_t c2r = make_rsrc(w.code2, w.nested ? 1024 : 0);
        hi = bload4(cr, (e >> 4) * 4);
        lo2 = bload4(cr, (e & 15) * 4);
        c2 = bload4(c2r, i * 4);
    }
    // LoRA T[m][lane] (dword loads, like the B rows below: no wait here)
    const rsrc_t tr = make_rsrc(lo.t, lora ? (a.M * lo.rank * 2 + 3) & ~int64_t(3) : 0);
    uint32_t tw[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) tw[m] = bload4(tr, (m * lo.rank + lane) * 2 & ~3);
    // this part's activations: token m, slot s holds elements 2048 (slot0 + s) + 32 lane .. + 31
    u32x4_t xr[SP][MT][4];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const rsrc_t xs = make_rsrc(a.act + m * a.ld_act, m < a.M ? K * 2 : 0);
#pragma unroll
        for (int sl = 0; sl < SP; ++sl)
#pragma unroll
            for (int q = 0; q < 4; ++q) xr[sl][m][q] = bload16(xs, (slot0 + sl) * 4096 + lane * 64 + q * 16);
    }
    __builtin_amdgcn_sched_barrier(0);  // the ring loads below stay behind these

    struct Slot {
        u32x4_t p;
        uint32_t qw;  // dword holding the block's uint8 absmax code (nested)
        float s;      // absmax2 scale (nested) or the fp32 absmax
    };
    Slot ring[RD][SP];
    uint32_t lbw[RD];  // dword holding the row's LoRA B value of this lane
    int lblk[SP];      // absmax block of this lane's bytes in a slot, relative to the row
#pragma unroll
    for (int sl = 0; sl < SP; ++sl) lblk[sl] = (2 * (1024 * (slot0 + sl) + 16 * lane)) >> w.bs_shift;
    const int last = nrows > 0 ? nrows - 1 : 0;
    auto load = [&](int j, int r) {
        const int rr = r < nrows ? r : last;
        const int64_t row = lrow0 + static_cast<int64_t>(rr) * gs;
#pragma unroll
        for (int sl = 0; sl < SP; ++sl) {
            const int byte = 1024 * (slot0 + sl) + 16 * lane;
            const int b = static_cast<int>(row) * kb + lblk[sl];
            ring[j][sl].p = bload16(wr.packed, static_cast<int>(row * khalf) + byte);
            ring[j][sl].qw = bload4(qr, b & ~3);
            ring[j][sl].s = __builtin_bit_cast(float, bload4(wr.s, (wr.nested ? b >> wr.bs2_shift : b) * 4));
        }
        lbw[j] = bload4(br, (static_cast<int>(row) * lo.rank + lane) * 2 & ~3);
    };
    // The first rows' loads go out before the table work, so their latency overlaps it; issued
    // by every wave (a padding group's reads row 0), so that the wait below retires the
    // activation loads on every path.
    // Row by row, in the loop's order (interleaved, the loop's wait counts inherit the worst
    // position a row's loads had here).
#pragma unroll
    for (int j = 0; j < RD; ++j) {
        load(j, j);
        __builtin_amdgcn_sched_barrier(0);
    }

    if (threadIdx.x < (kPrivate ? 512 : 256)) {  // write the tables (loaded at the top)
        const uint32_t v = static_cast<uint32_t>(round16<DT>(__builtin_bit_cast(float, hi))) |
                           (static_cast<uint32_t>(round16<DT>(__builtin_bit_cast(float, lo2))) << 16);
        if constexpr (kPrivate) {
            u32x4_t *dst = reinterpret_cast<u32x4_t *>(s_pair + e * 64 + (threadIdx.x & 1) * 32);
#pragma unroll
            for (int j = 0; j < 8; ++j) dst[j] = (u32x4_t){v, v, v, v};
        } else {
            s_pair[i] = v;
        }
        if (threadIdx.x < 256) s_code2[i] = w.nested ? __builtin_bit_cast(float, c2) : (i == 0 ? 1.0f : 0.0f);
    }
    __syncthreads();

    // Retire the activation loads (all but the ring's RD rows of loads, issued after them)
    // before the loop: left in flight into it, they make the compiler's wait counts for the
    // ring loads conservative down to zero.
    constexpr int kRingLoads = RD * (3 * SP + 1);
    static_assert(kRingLoads < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((kRingLoads & 0xF) | ((kRingLoads >> 4) << 14) | (0x7 << 4) | (0xF << 8));
    float tv[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const uint16_t h = static_cast<uint16_t>(tw[m] >> (((m * lo.rank + lane) & 1) * 16));
        tv[m] = (lane < lo.rank && m < a.M) ? to_f32<DT>(h) : 0.0f;
    }
    float res[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) res[m] = 0.0f;
    const char *pair = reinterpret_cast<const char *>(s_pair);
    const uint32_t lane4 = static_cast<uint32_t>(lane) * 4;
    // table entry of byte k of a packed dword: byte address 4 b (one copy), or 256 b + 4 lane
    // (lane4 in byte 0 and b in byte 1: one v_perm)
    auto entry = [&](uint32_t pw, int k) -> uint32_t {
        const uint32_t addr = kPrivate ? vperm(pw, lane4, 0x0C0C0400u | ((4u + k) << 8))
                                       : ((pw >> (8 * k)) & 0xFFu) * 4;
        return *reinterpret_cast<const uint32_t *>(pair + addr);
    };
    const float *code2 = s_code2;
    // Whole rounds of RD rows; the ring slot of a row past the range (a re-read of the last
    // row) is refilled but not computed.
    for (int r0 = 0; r0 < nrows; r0 += RD) {
#pragma unroll
        for (int j = 0; j < RD; ++j) {
            const int r = r0 + j;
            const int rr = r < nrows ? r : last;  // the row the ring holds
            if (r < nrows) {
            float acc[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
#pragma unroll
            for (int sl = 0; sl < SP; ++sl) {
                const Slot &sv = ring[j][sl];
                const int sh = ((static_cast<int>(lrow0 + rr * gs) * kb + lblk[sl]) & 3) * 8;
                const float sc = absmax_val(w, AbsIn{sv.s, (sv.qw >> sh) & 0xFFu}, code2);
                const uint32_t pw[4] = {sv.p.x, sv.p.y, sv.p.z, sv.p.w};
                uint32_t t[16];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    t[4 * d + 0] = entry(pw[d], 0);
                    t[4 * d + 1] = entry(pw[d], 1);
                    t[4 * d + 2] = entry(pw[d], 2);
                    t[4 * d + 3] = entry(pw[d], 3);
                }
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const u32x4_t xq = xr[sl][m][q];
                        d0 = dot2<DT>(t[4 * q + 0], xq.x, d0);
                        d1 = dot2<DT>(t[4 * q + 1], xq.y, d1);
                        d0 = dot2<DT>(t[4 * q + 2], xq.z, d0);
                        d1 = dot2<DT>(t[4 * q + 3], xq.w, d1);
                    }
                    acc[m] += (d0 + d1) * sc;
                }
            }
            {  // LoRA (branch-free: tv is zero without it, and lbw reads zero)
                const int be = static_cast<int>(lrow0 + rr * gs) * lo.rank + lane;
                const float bv = to_f32<DT>(static_cast<uint16_t>(lbw[j] >> ((be & 1) * 16)));
#pragma unroll
                for (int m = 0; m < MT; ++m) acc[m] += lscale * (tv[m] * bv);
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float tot = wave_sum(acc[m]);
                res[m] = lane == r ? tot : res[m];
            }
            }
            // The refill of ring slot j stays after the code that reads it and before the next
            // row's: hoisted, it needs copies of the slot that wait for every load in flight.
            __builtin_amdgcn_sched_barrier(0);
            load(j, r + RD);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    if (np > 1) {  // add the other parts' sums, in part order, into part 0's
#pragma unroll
        for (int m = 0; m < MT; ++m) s_part[wave][m][lane] = res[m];
        __syncthreads();
        if (part == 0) {
            for (int p = 1; p < np; ++p)
#pragma unroll
                for (int m = 0; m < MT; ++m) res[m] += s_part[wave + p][m][lane];
        }
    }
    if (part == 0 && lane < nrows) {
        const int64_t col = a.seg_off[seg] + gi + static_cast<int64_t>(lane) * gs;
        const float bias = a.bias ? to_f32<DT>(a.bias[col]) : 0.0f;
#pragma unroll
        for (int m = 0; m < MT; ++m)
            if (m < a.M) static_cast<uint16_t *>(a.out)[m * a.ld_out + col] = round16<DT>(res[m] + bias);
    }
}

// One workgroup of the input-gradient GEMM (as fwd_body).
template <int DT, int BP, int BM, int WP, int WM, int KG>
__device__ __forceinline__ void dx_body(const GemmArgs &a, const TileMap &tm, uint32_t blk,
                                        uint8_t *lds, float (*s_code2)[256]) {
    constexpr int NT = WP * WM * 64;  // threads of one k-group
    constexpr int TP = BP / WP / 32, TM = BM / WM / 32;
    static_assert(NT == 2 * BP, "dX weight tile mapping needs 2 threads per k column group");
    constexpr int NS = 2;  // LDS stages per k-group
    static_assert(KG == 1 || BP * BM * 4 <= stage_bytes<BP, BM, KG>(),
                  "the k-group sums fit in the staging tiles");
    auto sT = reinterpret_cast<uint8_t(*)[NS][(BP + BM) * ROWB]>(lds);

    const BlockTile bt = block_tile(a, blk);
    const int split = bt.split;
    const uint32_t tile = static_cast<uint32_t>(bt.tile);
    const uint32_t mtl = static_cast<uint32_t>(tm.m_tiles);
    const int64_t p0 = uniform64(tm.col0 + static_cast<int64_t>(tile / mtl) * BP);
    const int64_t m0 = uniform64(static_cast<int64_t>(tile % mtl) * BM);
    const int64_t K = a.K;
    const int64_t per = bt.nsplit > 1 ? a.per_split : a.total_steps;
    const int64_t s0 = uniform64(split * per);
    const int64_t s1 = uniform64(s0 + per < a.total_steps ? s0 + per : a.total_steps);

    for (int s = 0; s < a.nseg; ++s)
        for (int i = threadIdx.x; i < 256; i += KG * NT) s_code2[s][i] = code2_entry(a.w[s], i);

    const int wave_all = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int g = KG > 1 ? wave_all / (WP * WM) : 0;           // k-group
    const int wave = KG > 1 ? wave_all % (WP * WM) : wave_all;  // wave inside the group
    const int wp = wave % WP, wm = wave / WP;
    const int lane = threadIdx.x & 63;

    float16_t acc[TP][TM];
#pragma unroll
    for (int i = 0; i < TP; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = (float16_t){};

    // LoRA slabs: acc += A^T[k rows] . da[m rows]^T (reduction over the rank).
    if (split == 0 && g == 0) {
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
                    fb[j] = (m < a.M && lim > 0)
                                ? lora_row8(lo.da + m * lo.rank + k0 + kh, lim, lo.vec)
                                : (u32x4_t){0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int i = 0; i < TP; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j) acc[i][j] = mfma32<DT>(fa[i], fb[j], acc[i][j]);
            }
        }
    }

    uint8_t *sW[2] = {sT[g][0], sT[g][1]};
    uint8_t *sA[2] = {sT[g][0] + BP * ROWB, sT[g][1] + BP * ROWB};
    DxWeight<DT, BP> wt[2] = {};
    const rsrc_t ar = act_rsrc<BM>(a, m0);
    const rsrc_t ar0 = make_rsrc(a.act, 0);
    // the dY tile by LDS DMA, as the forward kernel's activation tile
    constexpr int CHA = BM * 8 / NT;
    static_assert(CHA >= 1 && BM * 8 % NT == 0, "dY rows split evenly over the waves");
    int adoff[CHA];
#pragma unroll
    for (int j = 0; j < CHA; ++j) {
        const int row = (wave * CHA + j) * 8 + (lane >> 3);
        adoff[j] = row * static_cast<int>(a.ld_act) * 2 + (((lane & 7) ^ ((row >> 1) & 7)) << 4);
    }
    const uint32_t lds_a =  // this wave's dY rows in the group's LDS stage 0
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t *)lds)) +
        (g * NS * (BP + BM) + BP + wave * CHA * 8) * ROWB;
    // every DMA is followed by exactly one weight register stage's 3 loads before this wait
    auto wait_dma = [] { asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); };
    __syncthreads();  // tables
    // The reduction range [s0, s1) walks the stacked segments in order; each segment runs the
    // forward kernel's pipeline (two weight register stages, two LDS stages, the next step's
    // dequant interleaved with the MFMAs and its dY tile sent by LDS DMA after the first
    // k-substep, no branches in the loop body, odd step after the loop) over the group's steps
    // b0 + g + KG v of the segment, with the segment's descriptor held in registers.  A
    // segment's partial last step (rows % 64 != 0) has its dY columns past the segment zeroed
    // in LDS once its DMA has landed (a branch and a barrier that the whole workgroup takes
    // when any group's step is such a step); rows past the weight dequantize from zero bytes
    // and meet those zeros.
    for (int seg = seg_of_step(a, s0); seg < a.nseg && a.step_start[seg] < s1; ++seg) {
        const int64_t first = a.step_start[seg];
        const int64_t b0 = first > s0 ? first : s0;
        const int64_t e0 = a.step_start[seg + 1] < s1 ? a.step_start[seg + 1] : s1;
        if (b0 >= e0) continue;
        const int64_t nv = (e0 - b0 + KG - 1) / KG;  // the same in every group
        const DevWeight w = a.w[seg];
        const WeightRsrc wr = weight_rsrc(w);
        const WAddr wa = dx_waddr<BP>(wr, p0, K);
        const int64_t col_base = a.seg_off[seg];
        const float *code2 = s_code2[seg];
        float code_r[16];
        load_code_sgpr(w.code, code_r);
        const Nf4HalfCodes hc = half_codes(code_r);
        auto dma_a = [&](int b, int64_t v) {  // dY columns of step v into LDS stage b
            const int64_t st = b0 + g + KG * v;
            const rsrc_t rs = KG > 1 && st >= e0 ? ar0 : ar;
            const int kb = static_cast<int>((col_base + (st - first) * BR) * 2);
            const uint32_t base = __builtin_amdgcn_readfirstlane(lds_a + b * (BP + BM) * ROWB);
#pragma unroll
            for (int j = 0; j < CHA; ++j) {
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                             :
                             : "s"(base + j * 8 * ROWB), "v"(adoff[j]), "s"(rs), "s"(kb)
                             : "memory", "m0");
            }
        };
        auto stage = [&](int b, int64_t v) { wt[b].load(wr, wa, (b0 + g + KG * v - first) * BR, K); };
        // After the DMA of step v into stage b has landed and the barrier: zero its columns past
        // the segment if step v is the segment's partial last step in any group.
        auto mask_lds = [&](int b, int64_t v) {
            bool any = false;
            int mine = BR;
#pragma unroll
            for (int gg = 0; gg < KG; ++gg) {
                const int64_t st = b0 + gg + KG * v;
                const int64_t left = w.rows - (st - first) * BR;
                const bool part = v < nv && st < e0 && left < BR;
                any = any || part;
                if (gg == g && part) mine = static_cast<int>(left);
            }
            if (!any) return;
            if (mine < BR) {
                for (int idx = threadIdx.x % NT; idx < BM * 8; idx += NT) {
                    const int row = idx >> 3, c = idx & 7;
                    const int k = mine - c * 8;  // valid elements of chunk c
                    if (k >= 8) continue;
                    u32x4_t *q = reinterpret_cast<u32x4_t *>(sA[b] + swz(row, c));
                    uint32_t mk[4];
#pragma unroll
                    for (int d = 0; d < 4; ++d)
                        mk[d] = ((2 * d < k) ? 0x0000ffffu : 0u) | ((2 * d + 1 < k) ? 0xffff0000u : 0u);
                    const u32x4_t x = *q;
                    *q = (u32x4_t){x.x & mk[0], x.y & mk[1], x.z & mk[2], x.w & mk[3]};
                }
            }
            __syncthreads();
        };
        __syncthreads();  // the previous segment's last MFMAs have read the LDS stages
        dma_a(0, 0);
        stage(0, 0);
        stage(1, 1);
        {
            const Nf4Table tb = make_table_half<DT>(hc, absmax_val(w, wt[0].abs, code2));
#pragma unroll
            for (int q = 0; q < 4; ++q) wt[0].store_part(sW[0], tb, hc.selbase, q);
        }
        wait_dma();
        __syncthreads();
        mask_lds(0, 0);
        int64_t v = 0;
        for (; v + 1 < nv; v += 2) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const Nf4Table tb = make_table_half<DT>(hc, absmax_val(w, wt[b ^ 1].abs, code2));
                mma_step_dx<DT, BP, TP, TM>(
                    acc, sW[b], sA[b], wp * (BP / WP), wm * (BM / WM), [&](int ks) {
                        wt[b ^ 1].store_part(sW[b ^ 1], tb, hc.selbase, ks);
                        if (ks == 0) {
                            dma_a(b ^ 1, v + b + 1);
                            stage(b, v + b + 2);
                        }
                    });
                wait_dma();
                __syncthreads();
                mask_lds(b ^ 1, v + b + 1);
            }
        }
        if (v < nv)
            mma_step_dx<DT, BP, TP, TM>(acc, sW[0], sA[0], wp * (BP / WP), wm * (BM / WM),
                                        [](int) {});
    }
    if constexpr (KG > 1) group_sum<TP, TM, KG, NT>(acc, &sT[0][0][0], g);
    if constexpr (stage_bytes<BP, BM, KG>() >= BM * BP * 2) {
        if (a.vec16_out && bt.nsplit == 1 && !a.bias && !a.accumulate) {
            epilogue_lds<DT, BP, BM, TP, TM, NT, KG>(a, acc, lds, p0, wp * (BP / WP), K, 0, m0,
                                                     wm * (BM / WM), g);
            return;
        }
    }
    if constexpr (BP == 128 && stage_bytes<BP, BM, KG>() >= BM * BP * 4) {
        if (a.vec16_out && bt.nsplit == 1) {
            epilogue_lds32<DT, BP, BM, TP, TM, NT, KG>(a, acc, lds, p0, wp * (BP / WP), K, 0, m0,
                                                       wm * (BM / WM), g);
            return;
        }
    }
    if constexpr (BP == 256 && KG == 1 && stage_bytes<BP, BM, KG>() >= BM * 512) {
        if (bt.nsplit > 1 && a.tail_cols % 4 == 0 && a.tail_col0 % 4 == 0) {
            partial_lds<BM, WM, TP, TM, NT>(a, acc, lds, p0, wp * (BP / WP), K, 0, m0,
                                        wm * (BM / WM), split);
            return;
        }
    }
    epilogue<DT, TP, TM, KG>(a, acc, p0 + wp * (BP / WP), K, 0, m0 + wm * (BM / WM), split,
                             bt.nsplit > 1, g);
}

template <int DT, int BP, int BM, int WP, int WM, int KG = 1>
__global__ __launch_bounds__(KG *WP *WM * 64) void dx_kernel(const GemmArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[stage_bytes<BP, BM, KG>()];
    __shared__ float s_code2[kMaxSeg][256];
    dx_body<DT, BP, BM, WP, WM, KG>(a, a.map[0], blockIdx.x, lds, s_code2);
}

// Two-part input-gradient launch (as fwd_head_tail_kernel): output columns of the first part
// in 256x256 tiles, the rest in 128x128 tiles with two k-groups.
template <int DT>
__global__ __launch_bounds__(512) void dx_head_tail_kernel(const GemmArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[stage_bytes<256, 256, 1>()];
    __shared__ float s_code2[kMaxSeg][256];
    const uint32_t b0 = static_cast<uint32_t>(a.blocks0);
    if (blockIdx.x < b0)
        dx_body<DT, 256, 256, 2, 4, 1>(a, a.map[0], blockIdx.x, lds, s_code2);
    else
        dx_body<DT, 128, 128, 2, 2, 2>(a, a.map[1], blockIdx.x - b0, lds, s_code2);
}

// Split reduction over the tail columns [col0, col0 + n_out):
// out[m][col0 + c] = sum_s partial[s][m][c] (+ bias[col0 + c]) (+ out[m][col0 + c]) in split
// order (deterministic).  Grid: x = groups of 1024 columns (4 per thread), y = rows.
template <int DT>
__global__ __launch_bounds__(256) void split_reduce_kernel(const float *partial, int splits,
                                                           int64_t M, int64_t n_out, int64_t col0,
                                                           const uint16_t *bias, uint16_t *out,
                                                           int64_t ld_out, int accumulate,
                                                           int vec) {
    const int64_t c0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (c0 >= n_out) return;
    const int64_t total = M * n_out;
    const int nc = n_out - c0 < 4 ? static_cast<int>(n_out - c0) : 4;
    if (bias) bias += col0;
    out += col0;
    for (int64_t m = blockIdx.y; m < M; m += gridDim.y) {
        const int64_t base = m * n_out + c0;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (vec && nc == 4) {
            // the loads of 8 splits go out together (the partials come from other XCDs' writes,
            // one memory latency each: issued one by one they cost a latency per split), then
            // are added in split order
            constexpr int U = 8;
            for (int s0 = 0; s0 < splits; s0 += U) {
                float4_t t[U];
#pragma unroll
                for (int u = 0; u < U; ++u)
                    t[u] = s0 + u < splits
                               ? *reinterpret_cast<const float4_t *>(partial + (s0 + u) * total + base)
                               : (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    if (s0 + u >= splits) break;
                    v[0] += t[u].x;
                    v[1] += t[u].y;
                    v[2] += t[u].z;
                    v[3] += t[u].w;
                }
            }
        } else {
            for (int s = 0; s < splits; ++s)
                for (int q = 0; q < nc; ++q) v[q] += partial[s * total + base + q];
        }
        uint16_t *dst = out + m * ld_out + c0;
        for (int q = 0; q < nc; ++q) {
            if (bias) v[q] += to_f32<DT>(bias[c0 + q]);
            if (accumulate) v[q] += to_f32<DT>(dst[q]);
        }
        if (vec && nc == 4) {
            u32x2_t o;
            o.x = pack2<DT>(v[0], v[1]);
            o.y = pack2<DT>(v[2], v[3]);
            *reinterpret_cast<u32x2_t *>(dst) = o;
        } else {
            for (int q = 0; q < nc; ++q) dst[q] = from_f32<DT>(v[q]);
        }
    }
}

// ------------------------------------------------------------------------------ host side

struct Plan {
    int cfg;       // 0: 256x256 tile / 8 waves, 1: 128x128 tile / 4 waves, 3: 128x128 tile /
                   // two k-groups of 4 waves, 2: small-M path,
                   // 4: decode path (M <= 16), 6: row streaming (M <= 2), 7: skinny path
                   // (2 < M <= 64)
    int bp, bm;
    int splits;    // reduction splits of the tail tiles
    int64_t tiles;
    int waves;     // small-M and decode paths: waves per workgroup
    int64_t tail_start;  // first split tile (tiles before it run whole)
    // > 0: two launches, whole rounds of 256x256 tiles over the first head_ptiles p-tiles (rows
    // of the stacked weights forward, columns of dX backward), then the rest in unsplit 128x128
    // tiles of tiling `cfg` (1 or 3); `tiles` then counts the second launch's tiles (estimate).
    int64_t head_ptiles;
    int rows_g = 0;  // row-streaming path: row groups per workgroup
    int dks = 0;     // skinny path: super-step depth (128 or 256)
    int fx = 0;      // skinny path: LoRA down-projections computed in the launch

    int64_t blocks() const { return tail_start + (tiles - tail_start) * splits; }
};

// The small-M forward path takes M <= kGemvMaxM (32 activation rows: one MFMA B operand).  Its workgroups own 32 weight rows and their share of the reduction, spread over
// 16 waves (8 with two activation fragments) while there are at most as many workgroups as
// CUs, else 4 waves with several steps each.  Long reductions over few row tiles are split over
// workgroups.
constexpr int64_t kGemvMaxM = 32;

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
        // The fused main loop needs each 64-wide step of a weight row inside one absmax block,
        // and power-of-two block sizes (shifts instead of divisions in the main loop).
        if (ws[i].blocksize % BR != 0 || g.K % ws[i].blocksize != 0) return NF4_ERR_UNSUPPORTED;
        if (log2_exact(ws[i].blocksize) < 0) return NF4_ERR_UNSUPPORTED;
        if (ws[i].nested && log2_exact(ws[i].blocksize2) < 0) return NF4_ERR_UNSUPPORTED;
        if (!aligned(ws[i].packed, 16)) return NF4_ERR_UNSUPPORTED;
        g.w[i] = to_dev(ws[i]);
    }
    if (g.K % BR != 0 || ld_act % 8 != 0 || !aligned(act, 16)) return NF4_ERR_UNSUPPORTED;
    // Main-loop loads use 32-bit byte offsets inside buffer resources: a 256-row activation
    // window and each weight (plus one tile of rows past its end) must stay below 2 GiB.
    if (ld_act >= (int64_t(1) << 21)) return NF4_ERR_UNSUPPORTED;
    for (int i = 0; i < nw; ++i) {
        const int64_t n = (ws[i].rows + 256) * ws[i].cols;
        if (n / 2 >= (int64_t(1) << 31) || (n / ws[i].blocksize) * 4 >= (int64_t(1) << 31))
            return NF4_ERR_UNSUPPORTED;
    }
    return NF4_OK;
}

// Tile and split choice by a cost model whose constants were measured on MI355X (fp16, M = 2048,
// every Qwen2.5-1.5B projection, each plan timed): one 64-deep step of a 256x256 tile takes
// ~2.45 us with one workgroup per CU; a 128x128 step ~1.4 us with two workgroups per CU.
// Workgroups run in rounds of 256 (256x256) or 512 (128x128); a last 128x128 round of at most
// 256 workgroups runs one per CU at the single-workgroup speed (~1.15 us per step).  A single
// round of 128x128 tiles with one workgroup per CU costs ~7.8 us + 0.93 us per step with 4 waves
// and ~8.5 us + 0.75 us per step with two k-groups of 4 waves (timed over K).  Split-K adds
// the fp32 partial round trip (written by the GEMM, read back by the reduction) at ~5 TB/s plus
// ~12 us of reduction launch and tail.  The larger tile needs 4x fewer dequant instructions per
// MFMA, which the step times already contain.
constexpr int kMaxSplits = 16;
constexpr double kLaunchGap = 2.0;  // us between two dependent launches on one stream

// Time of a plan: workgroups are dispatched in order into `slots` places (one per CU for the
// 256x256 tile, two for 128x128).  The whole tiles run in rounds; the split tail tiles' shorter
// workgroups first fill the places the last whole round leaves free, then run in rounds of
// their own.  A split also pays the fp32 partial round trip and the reduction launch.
double plan_cost(int cfg, int64_t tiles, int64_t mt, int64_t tail_start, int splits,
                 int64_t steps, int64_t m) {
    const int64_t slots = cfg == 0 ? kCUs : 2 * kCUs;
    const int64_t bp = cfg == 0 ? 256 : 128;
    const int64_t full = splits > 1 ? tail_start : tiles;
    const int64_t tail_blocks = splits > 1 ? (tiles - tail_start) * splits : 0;
    const int64_t per = (steps + splits - 1) / splits;
    const double split_cost =
        splits > 1 ? 2.0 * double(splits) * double(m) * double((tiles - tail_start) / mt) *
                             double(bp) * 4.0 / 5.0e6 + 12.0
                   : 0.0;
    if (cfg == 3 || (cfg == 1 && full + tail_blocks <= kCUs)) {
        // 128x128 tiles, one workgroup per CU in a single round: fixed cost (launch, tables,
        // first loads, epilogue) plus the longest workgroup's steps, measured with 4 waves and
        // with two k-groups of 4 waves; the k-groups take no more than one round
        if (full + tail_blocks > kCUs) return 1e30;
        const double st = double(full > 0 ? steps : per);
        return (cfg == 3 ? 0.75 * st + 8.5 : 0.93 * st + 7.8) + split_cost;
    }
    const double t_step = cfg == 0 ? 2.45 : 1.4;
    const int64_t rounds = (full + slots - 1) / slots;
    double c = double(rounds) * double(steps) * t_step + 1.0;
    if (cfg == 1 && full > kCUs && full % slots != 0 && full % slots <= kCUs && tail_blocks == 0)
        c -= double(steps) * (t_step - 1.15);  // the last round alone on its CUs
    const int64_t free_slots = rounds * slots - full;
    if (tail_blocks > free_slots)
        c += double((tail_blocks - free_slots + slots - 1) / slots) * double(per) * t_step;
    return c + split_cost;
}

// `ws_cap` >= 0 (input-gradient plans only, `out_cols` = K): leave out split plans whose fp32
// partials, splits x M x (columns from the tail's first p tile to K), exceed ws_cap bytes.
Plan make_plan(int64_t m, int64_t big, int64_t small, int64_t steps, int max_splits = kMaxSplits,
               int64_t out_cols = 0, int64_t ws_cap = -1) {
    Plan best{};
    double best_cost = 0.0;
    for (int cfg : {0, 1, 3}) {
        const int64_t tiles = cfg == 0 ? big : small;
        const int64_t mt = (m + (cfg == 0 ? 255 : 127)) / (cfg == 0 ? 256 : 128);
        const int64_t bp = cfg == 0 ? 256 : 128;
        for (int s = 1; s <= max_splits; ++s) {
            const int64_t per = (steps + s - 1) / s;
            if (s > 1 && (s - 1) * per >= steps) break;  // no empty split
            // the split tail starts at a p-tile boundary (a column range of the output)
            for (int64_t ts = 0; ts < (s > 1 ? tiles : 1); ts += mt) {
                if (s > 1 && ws_cap >= 0 &&
                    int64_t(s) * m * (out_cols - (ts / mt) * bp) * 4 > ws_cap)
                    continue;
                const double c = plan_cost(cfg, tiles, mt, ts, s, steps, m);
                if (best.splits == 0 || c < best_cost) {
                    best = Plan{cfg, cfg == 0 ? 256 : 128, cfg == 0 ? 256 : 128, s, tiles, 0,
                                s > 1 ? ts : tiles};
                    best_cost = c;
                }
            }
        }
    }
    // Head + tail: r whole rounds of 256x256 tiles, then the rows (columns) left in one
    // unsplit launch of 128x128 tiles; each 256-row p-tile of the head removes two 128-row
    // p-tiles from the tail (an estimate where a segment ends inside a p-tile).
    const int64_t mt0 = (m + 255) / 256, mt1 = (m + 127) / 128;
    for (int64_t r = 1; r * kCUs < big; ++r) {
        const int64_t hp = r * kCUs / mt0;
        const int64_t tail = small - 2 * hp * mt1;
        if (hp <= 0 || hp * mt0 >= big || tail <= 0) continue;
        const double head = plan_cost(0, hp * mt0, mt0, hp * mt0, 1, steps, m);
        for (int cfg : {1, 3}) {
            const double c = head + plan_cost(cfg, tail, mt1, tail, 1, steps, m) + kLaunchGap;
            if (c < best_cost) {
                best = Plan{cfg, 128, 128, 1, tail, 0, tail, hp};
                best_cost = c;
            }
        }
    }
    return best;
}

Plan plan_gemv(int64_t m, const nf4_weight *ws, int nw) {
    int64_t tiles = 0;
    for (int i = 0; i < nw; ++i) tiles += (ws[i].rows + 31) / 32;
    const int64_t steps = ws[0].cols / BR;
    int waves = tiles > kCUs ? 4 : 16;
    while (waves > 4 && waves > steps) waves /= 2;
    // few row tiles and a long reduction: split it over workgroups (fp32 partials + the
    // fixed-order reduction) so that more CUs dequantize, keeping >= 2 steps per wave
    int64_t splits = 1;
    if (tiles < kCUs / 2) {
        splits = kCUs / tiles;
        const int64_t by_steps = steps / (2 * waves);
        if (splits > by_steps) splits = by_steps;
        if (splits > kMaxSplits) splits = kMaxSplits;
        if (splits < 1) splits = 1;
        while (splits > 1 && (splits - 1) * ((steps + splits - 1) / splits) >= steps) --splits;
    }
    return Plan{2, 32, 32, static_cast<int>(splits), tiles, waves, splits > 1 ? 0 : tiles};
}

// Decode path: waves per 16-row tile, the most (up to 8) that keep the whole launch resident
// (kDecodeWavesPerSimd waves per SIMD) and give every wave at least three super-steps (fewer
// make the cross-wave reduction and the prefetch ramp dominate).  16 waves measured slower than
// 8 where they were allowed (the down projections at M <= 8: 28-layer forward 2-5 % slower).
Plan plan_decode(const nf4_weight *ws, int nw) {
    int64_t tiles = 0;
    for (int i = 0; i < nw; ++i) tiles += (ws[i].rows + 15) / 16;
    const int64_t ss = ws[0].cols / DK;
    int waves = 8;
    while (waves > 1 && (tiles * waves > 4 * kDecodeWavesPerSimd * kCUs || 3 * waves > ss)) waves /= 2;
    return Plan{4, 16, 16, 1, tiles, waves, tiles};
}

// Forward path by token count: the decode kernel up to 16 tokens (K a multiple of 128), the
// small-M kernel up to 32, the tiled GEMMs (with split-K) from 33 on.  Measured on 4-layer
// Qwen2.5-1.5B / -7B stacks (forward per layer, HIP graph replay): at M = 20-32 the small-M
// kernel is 10-22 % faster on the 1.5B stack and within -6..+6 % on the 7B stack; at M = 40-64
// the tiled plans are up to 12 % faster per layer (the 7B down projection, K = 18944, most).
// A tiling pinned by the caller: tile shape `tile` (0, 1 or 3 as Plan::cfg) with every tile's
// reduction split `splits` ways (1: none); an empty last split is refused (splits = 0 returned).
Plan pinned_plan(int tile, int splits, int64_t big, int64_t small, int64_t steps) {
    if ((tile != 0 && tile != 1 && tile != 3) || splits < 1 || splits > kMaxSplits) return Plan{};
    const int64_t per = (steps + splits - 1) / splits;
    if (splits > 1 && (splits - 1) * per >= steps) return Plan{};
    const int b = tile == 0 ? 256 : 128;
    const int64_t tiles = tile == 0 ? big : small;
    return Plan{tile, b, b, splits, tiles, 0, splits > 1 ? 0 : tiles};
}

// Row-streaming path (M <= 2): K parts of one 1 KB slot when a row takes one slot or 3 to
// kRowsMaxParts slots (the 1.5B down projection, 5 slots: 5 one-slot parts ran 19 % faster than
// 3 two-slot parts, which left 102 CUs idle and read 27 % past the rows), of two slots
// otherwise (the 7B rows of 2 slots keep one part and the kernel's 64-copy table); workgroups
// of G row groups x np parts (8 waves for a single one-slot part, at most 16 otherwise: the
// 64-copy table is filled once per CU), and the fewest rows per group that still fit the
// launch in one round of workgroups at 4 waves per SIMD (at most 64: one result lane each).  Plan::tiles counts row groups, Plan::waves holds the rows per group, Plan::bp the
// slots per part, Plan::bm the tokens per wave (1 or 2), Plan::splits the parts and
// Plan::rows_g the groups per workgroup.  From 3 tokens on the decode kernel's MFMA path is
// faster (its dequant is shared by the tokens).
Plan plan_rows(int64_t m, const nf4_weight *ws, int nw) {
    const int mt = m <= 1 ? 1 : 2;
    const int64_t ni = (ws[0].cols / 2 + 1023) / 1024;
    const int sp = ni == 1 || (ni > 2 && ni <= kRowsMaxParts) ? 1 : 2;
    const int np = static_cast<int>((ni + sp - 1) / sp);
    const int groups_per_wg = sp == 1 && np == 1 ? 8 : kRowsMaxWaves / np;
    const int wg_per_cu = kRowsMaxWaves / (np * groups_per_wg) > 1 ? kRowsMaxWaves / (np * groups_per_wg) : 1;
    int64_t rows = 0;
    for (int i = 0; i < nw; ++i) rows += ws[i].rows;
    const int64_t slots = static_cast<int64_t>(kCUs) * wg_per_cu * groups_per_wg;
    int64_t rpw = (rows + slots - 1) / slots;
    if (rpw < 1) rpw = 1;
    if (rpw > kRowsMaxRows) rpw = kRowsMaxRows;
    int64_t groups = 0;  // padded to whole workgroups per segment
    for (int i = 0; i < nw; ++i)
        groups += ((ws[i].rows + rpw - 1) / rpw + groups_per_wg - 1) / groups_per_wg * groups_per_wg;
    Plan p{6, sp, mt, np, groups, static_cast<int>(rpw), 0, 0};
    p.rows_g = groups_per_wg;
    return p;
}

bool rows_ok(int64_t m, const nf4_weight *ws, int nw) {
    const int64_t ni = (ws[0].cols / 2 + 1023) / 1024;
    if (m > kRowsMaxM || ni > 2 * kRowsMaxParts) return false;
    for (int i = 0; i < nw; ++i)
        if (!aligned(ws[i].absmax, 4)) return false;  // absmax codes are read as aligned dwords
    // 32-bit byte offsets: a wave reads up to 16 KB past the start of its last row
    for (int i = 0; i < nw; ++i)
        if (ws[i].rows * (ws[i].cols / 2) + 16 * 1024 >= (int64_t(1) << 31)) return false;
    return true;
}

// Skinny path (2 < M <= 64, K a multiple of 128): MT = 16-token groups, the workgroup shape
// RT row tiles x KP k-parts (8 waves), the super-step DKS and the reduction splits S from a cost
// model calibrated on the box with the weights streaming from HBM (every Qwen2.5-1.5B and -7B
// projection at M = 8 .. 64 and every split of the down projections, each shape's weights
// replicated past the 256 MB Infinity Cache; 276 timed points, mean error 5 %):
//   t = 3.57 us + 1.41 us per round of workgroups (ceil(workgroups x S / CUs))
//       + 0.0424 us (DKS 128) or 0.0357 us (DKS 256) per 1000 weight elements the busiest CU
//       holds, counting a k-part's idle super-steps (rounds x 16 RT x KP x ceil(K / DKS / S /
//       KP) x DKS), + 0.0087 us per 1000 of them when the kernel's registers or LDS leave one
//       workgroup per CU (skinny_slots), + 0.0056 us per 1000 for each 16-token group past the
//       first, + 0.052 us per MB of activations the workgroups read (each reads X over its part
//       of K)
//       + with S > 1: 2.4 us for the reduction launch (3.89 us before its loads of 8 splits
//       went out together; re-timed: 1.5B down at M = 8 11.4 us with 8 splits against 12.7 us
//       unsplit, 7B gate|up at M = 64 56.3 us with 2 splits against 57.5 us, 7B o at M = 64
//       15.4 against 16.3) + 0.223 us per MB of fp32 partials (8 S M N bytes: written, then
//       read back); a split holds at least 8 super-steps (shorter
//       ones measured slower than the model says: 1.5B down at M = 64, 14 splits 18.5 us, 8
//       splits 16.1 us).
// DKS = 256 only for one token group: with more its longer-lived registers cost a workgroup
// per CU (gate|up of Qwen2.5-7B at M = 24: 42 us against 36 us at DKS = 128).  The activation
// stages (2 x KP x 16 MT tokens x DKS x 2 bytes) must fit in LDS and a k-part of a split hold
// two super-steps.  Splits serve the long reductions over few rows (down projections), whose
// row tiles alone leave most CUs idle.  Plan::bp holds the rows per workgroup (16 RT),
// Plan::waves KP, Plan::bm 16 MT, Plan::dks DKS, Plan::splits S (tail_start 0: every tile
// split); the cost (us) is returned through `cost`.
constexpr bool skinny_fits(int kp, int mt, int dks) { return kp * mt * dks <= 2048; }

// Workgroups per CU that a skinny kernel's registers and LDS allow (the compiler's register
// counts for gfx950: 145 or more VGPRs leave 3 or fewer waves per SIMD, one 8-wave workgroup;
// tests/test_skinny_occupancy.py checks this table against the compiled kernels).
constexpr int skinny_slots(int mt, int rt, int dks) {
    return (dks == 256 && rt <= 2) || (mt == 2 && rt == 1) || (mt == 4 && rt <= 4) ? 1 : 2;
}

// fx_only: only plans that can compute a LoRA down-projection of rank <= 16 in the launch (one
// split, the stages 16 rows taller).
Plan plan_skinny(int64_t m, const nf4_weight *ws, int nw, double *cost = nullptr,
                 bool fx_only = false) {
    const int mt = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    const int64_t K = ws[0].cols;
    int64_t n_out = 0;
    for (int i = 0; i < nw; ++i) n_out += ws[i].rows;
    static constexpr int kShapes[4][2] = {{8, 1}, {4, 2}, {2, 4}, {1, 8}};
    Plan best{};
    double best_t = 1e30;
    for (const int dks : {256, 128}) {
        if (K % dks != 0 || (dks == 256 && mt > 1)) continue;
        const int64_t ss = K / dks;
        const double per_elem = dks == 256 ? 0.0357 : 0.0424;
        for (const auto &sh : kShapes) {
            const int rt = sh[0], kp = sh[1];
            if (!skinny_fits(kp, mt + (fx_only ? 1 : 0), dks)) continue;
            int64_t wgs = 0;
            for (int i = 0; i < nw; ++i) wgs += (ws[i].rows + 16 * rt - 1) / (16 * rt);
            for (const int sp_try : {1, 2, 4, 8, 16}) {
                const int64_t sps = (ss + sp_try - 1) / sp_try;  // super-steps per split
                if ((kp > 1 && sps < 2 * kp) || (sp_try > 1 && sps < 8)) break;
                const int sp = static_cast<int>((ss + sps - 1) / sps);  // no empty last split
                if (fx_only && (sp > 1 || mt > 2)) break;
                const int64_t per = (sps + kp - 1) / kp;
                const double rounds = double((wgs * sp + kCUs - 1) / kCUs);
                const double busy = rounds * 16.0 * rt * kp * per * dks / 1000.0;
                const double x_mb = double(wgs) * double(m) * double(K) * 2.0 / 1e6;
                const double one_wg = skinny_slots(mt, rt, dks) == 1 ? 0.0087 : 0.0;
                double t = 3.57 + 1.41 * rounds + busy * (per_elem + one_wg + 0.0056 * (mt - 1)) +
                           0.052 * x_mb;
                if (sp > 1) t += 2.4 + 0.223 * 8.0 * sp * double(m) * double(n_out) / 1e6;
                if (t < best_t) {
                    best = Plan{7, 16 * rt, 16 * mt, sp, wgs, kp, sp > 1 ? 0 : wgs};
                    best.dks = dks;
                    best_t = t;
                }
            }
        }
    }
    if (cost) *cost = best_t;
    return best;
}

// The decode kernel's time (one workgroup per 16 rows, K split over its waves): 5.26 us +
// 0.0637 us per 1000 elements of the busiest CU (+ 0.018 above 8 tokens); calibrated like the
// skinny model, its fixed part raised by the 1 us that streaming the weights from HBM added to
// its launches.
double decode_cost(int64_t m, const nf4_weight *ws, int nw) {
    int64_t t16 = 0;
    for (int i = 0; i < nw; ++i) t16 += (ws[i].rows + 15) / 16;
    const double busiest = double((t16 + kCUs - 1) / kCUs) * 16.0 * double(ws[0].cols) / 1000.0;
    return 5.26 + busiest * (m <= 8 ? 0.0637 : 0.0818);
}

// A skinny plan that can compute LoRA down-projections of rank <= 16 in its own launch: one
// reduction split (T needs all of K), at most two token groups, and the stages hold 16 more
// rows per k-part.  (With four token groups the plans that fit, 1 or 2 k-parts, measured
// slower than the best plan plus a separate launch: 7B q|k|v at M = 64 29.1 vs 26.6 us.)
bool skinny_fx_ok(const Plan &p, int xa_rank) {
    const int mt = p.bm / 16;
    return p.cfg == 7 && xa_rank >= 1 && xa_rank <= 16 && p.splits == 1 && mt <= 2 &&
           skinny_fits(p.waves, mt + 1, p.dks);
}

// A standalone LoRA down-projection launch (nf4_lora_xa_multi at up to 64 tokens: one
// workgroup per adapter, A row and 8 tokens), timed on the box back to back in a graph (the gap
// between launches included): 3.1 us at K = 1536, 4.2 us at K = 3584, at every token count to
// 64; + 0.5 us of margin.
double xa_launch_cost(int64_t k) { return 2.8 + 0.00054 * double(k); }
constexpr double kFxCost = 2.0;

// The skinny plan for the call: when it has LoRA down-projections to compute (xa_rank > 0: rank
// of the largest), the best plan plus their own launch against the best plan that computes
// them itself.  Either has no workspace when the plan without them has none, so the workspace
// query, which does not see the adapters, stays valid.
Plan choose_skinny(int64_t m, const nf4_weight *ws, int nw, int xa_rank, double *cost) {
    double t = 0;
    Plan p = plan_skinny(m, ws, nw, &t);
    if (xa_rank > 0 && t < 1e29) {
        // computing T in the launch adds ~2 us to it (7B q|k|v at M = 8: 12.8 vs 10.6 us)
        t += skinny_fx_ok(p, xa_rank) ? kFxCost : xa_launch_cost(ws[0].cols);
        double tf = 0;
        const Plan pf = plan_skinny(m, ws, nw, &tf, true);
        if (xa_rank <= 16 && tf + kFxCost < t) {
            p = pf;
            t = tf + kFxCost;
        }
    }
    *cost = t;
    return p;
}

// The skinny path takes 2 < M <= 64 with K a multiple of 128; at M <= 16 it also has to beat
// the decode kernel's modelled time (plus the LoRA down-projections' own launch, which the
// decode kernel never folds).
bool skinny_ok(int64_t m, const nf4_weight *ws, int nw, int xa_rank) {
    if (m <= 2 || m > kSkinnyMaxM || ws[0].cols % DK != 0) return false;
    double t = 0;
    choose_skinny(m, ws, nw, xa_rank, &t);
    if (t >= 1e29) return false;  // no workgroup shape fits
    if (m > kDecodeMaxM) return true;
    return t < decode_cost(m, ws, nw) + (xa_rank > 0 ? xa_launch_cost(ws[0].cols) : 0.0);
}

// rows_allowed: the row-streaming path's operand alignment holds (LoRA T and B read as dwords).
// xa_rank: the call's LoRA adapters ask for their down-projections (rank of the largest), which
// only moves the choice between the skinny and decode paths (neither needs a workspace).
Plan plan_fwd(int64_t m, const nf4_weight *ws, int nw, int tile = -1, int splits = 1,
              bool rows_allowed = true, int xa_rank = 0) {
    if (tile < 0 && rows_allowed && rows_ok(m, ws, nw)) return plan_rows(m, ws, nw);
    if (tile < 0 && skinny_ok(m, ws, nw, xa_rank)) {
        double t = 0;
        return choose_skinny(m, ws, nw, xa_rank, &t);
    }
    if (tile < 0 && m <= kDecodeMaxM && ws[0].cols % DK == 0) return plan_decode(ws, nw);
    if (tile < 0 && m <= kGemvMaxM) return plan_gemv(m, ws, nw);
    int64_t big = 0, small = 0;
    for (int i = 0; i < nw; ++i) {
        big += (ws[i].rows + 255) / 256;
        small += (ws[i].rows + 127) / 128;
    }
    big *= (m + 255) / 256;
    small *= (m + 127) / 128;
    if (tile >= 0) return pinned_plan(tile, splits, big, small, ws[0].cols / BR);
    return make_plan(m, big, small, ws[0].cols / BR);
}

Plan plan_dx(int64_t m, const nf4_weight *ws, int nw, int tile = -1, int splits = 1,
             int64_t ws_cap = -1) {
    int64_t steps = 0;
    for (int i = 0; i < nw; ++i) steps += (ws[i].rows + BR - 1) / BR;
    const int64_t K = ws[0].cols;
    const int64_t big = ((K + 255) / 256) * ((m + 255) / 256);
    const int64_t small = ((K + 127) / 128) * ((m + 127) / 128);
    if (tile >= 0) return pinned_plan(tile, splits, big, small, steps);
    return make_plan(m, big, small, steps, kMaxSplits, K, ws_cap);
}

// false: no kernel of this shape (the planner never asks for one)
template <int DT, int MT, int DKS, bool FX>
bool launch_skinny_d(const GemmArgs &g, int rt, dim3 grid, hipStream_t st) {
    const dim3 block(512);
    if constexpr (skinny_fits(1, MT + FX, DKS)) {
        if (rt == 8) {
            hipLaunchKernelGGL((skinny_kernel<DT, MT, 8, 1, DKS, FX>), grid, block, 0, st, g);
            return true;
        }
    }
    if constexpr (skinny_fits(2, MT + FX, DKS)) {
        if (rt == 4) {
            hipLaunchKernelGGL((skinny_kernel<DT, MT, 4, 2, DKS, FX>), grid, block, 0, st, g);
            return true;
        }
    }
    if constexpr (skinny_fits(4, MT + FX, DKS)) {
        if (rt == 2) {
            hipLaunchKernelGGL((skinny_kernel<DT, MT, 2, 4, DKS, FX>), grid, block, 0, st, g);
            return true;
        }
    }
    if constexpr (skinny_fits(8, MT + FX, DKS)) {
        if (rt == 1) {
            hipLaunchKernelGGL((skinny_kernel<DT, MT, 1, 8, DKS, FX>), grid, block, 0, st, g);
            return true;
        }
    }
    return false;
}

template <int DT, int MT>
bool launch_skinny(const GemmArgs &g, const Plan &p, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(p.blocks()));
    if constexpr (MT == 1) {  // the planner takes 256-deep super-steps for one token group only
        if (p.dks == 256)
            return p.fx ? launch_skinny_d<DT, MT, 256, true>(g, p.bp / 16, grid, st)
                        : launch_skinny_d<DT, MT, 256, false>(g, p.bp / 16, grid, st);
    }
    if constexpr (MT <= 2) {  // T in the launch: at most two token groups
        if (p.fx) return p.dks == 128 && launch_skinny_d<DT, MT, 128, true>(g, p.bp / 16, grid, st);
    }
    if (p.fx) return false;
    if (p.dks == 128) return launch_skinny_d<DT, MT, 128, false>(g, p.bp / 16, grid, st);
    return false;
}

template <int DT>
int launch_fwd(const GemmArgs &g, const Plan &p, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(p.blocks()));
    if (p.cfg == 7) {
        const bool ok = p.bm == 16 ? launch_skinny<DT, 1>(g, p, st)
                        : p.bm == 32 ? launch_skinny<DT, 2>(g, p, st)
                                     : launch_skinny<DT, 4>(g, p, st);
        if (!ok) return NF4_ERR_UNSUPPORTED;
    } else if (p.cfg == 4) {
        const dim3 block(p.waves * 64);
        if (p.waves == 8) hipLaunchKernelGGL((decode_kernel<DT, 8>), grid, block, 0, st, g);
        else if (p.waves == 4) hipLaunchKernelGGL((decode_kernel<DT, 4>), grid, block, 0, st, g);
        else if (p.waves == 2) hipLaunchKernelGGL((decode_kernel<DT, 2>), grid, block, 0, st, g);
        else hipLaunchKernelGGL((decode_kernel<DT, 1>), grid, block, 0, st, g);
    } else if (p.cfg == 2) {
        const dim3 block(p.waves * 64);
        if (p.waves == 16) hipLaunchKernelGGL((gemv_kernel<DT, 1, 16>), grid, block, 0, st, g);
        else if (p.waves == 8) hipLaunchKernelGGL((gemv_kernel<DT, 1, 8>), grid, block, 0, st, g);
        else hipLaunchKernelGGL((gemv_kernel<DT, 1, 4>), grid, block, 0, st, g);
    } else if (p.cfg == 0) {
        hipLaunchKernelGGL((fwd_rw_kernel<DT>), grid, dim3(512), 0, st, g);
    }
    else if (p.cfg == 3)
        hipLaunchKernelGGL((fwd_kernel<DT, 128, 128, 2, 2, 0, 2>), grid, dim3(512), 0, st, g);
    else
        hipLaunchKernelGGL((fwd_kernel<DT, 128, 128, 2, 2>), grid, dim3(256), 0, st, g);
    return status_of(hipGetLastError());
}

template <int DT, int EPI>
int launch_paired(const GemmArgs &g, const Plan &p, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(p.blocks()));
    if (p.cfg == 0) {
        hipLaunchKernelGGL((fwd_kernel<DT, 256, 256, 2, 4, EPI>), grid, dim3(512), 0, st, g);
    }
    else if (p.cfg == 3)
        hipLaunchKernelGGL((fwd_kernel<DT, 128, 128, 2, 2, EPI, 2>), grid, dim3(512), 0, st, g);
    else
        hipLaunchKernelGGL((fwd_kernel<DT, 128, 128, 2, 2, EPI>), grid, dim3(256), 0, st, g);
    return status_of(hipGetLastError());
}

template <int DT>
int launch_dx(const GemmArgs &g, const Plan &p, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(p.blocks()));
    if (p.cfg == 0)
        hipLaunchKernelGGL((dx_kernel<DT, 256, 256, 2, 4>), grid, dim3(512), 0, st, g);
    else if (p.cfg == 3)
        hipLaunchKernelGGL((dx_kernel<DT, 128, 128, 2, 2, 2>), grid, dim3(512), 0, st, g);
    else
        hipLaunchKernelGGL((dx_kernel<DT, 128, 128, 2, 2>), grid, dim3(256), 0, st, g);
    return status_of(hipGetLastError());
}

template <int DT>
int launch_reduce(const GemmArgs &g, int splits, hipStream_t st) {
    const int64_t cols = (g.tail_cols + 1023) / 1024;
    const int64_t rows = g.M < 65535 ? g.M : 65535;
    const int vec = g.tail_cols % 4 == 0 && g.tail_col0 % 4 == 0 && g.ld_out % 4 == 0 &&
                    aligned(g.out, 8) && aligned(g.partial, 16);
    hipLaunchKernelGGL(split_reduce_kernel<DT>,
                       dim3(static_cast<unsigned>(cols), static_cast<unsigned>(rows)), dim3(256),
                       0, st, g.partial, splits, g.M, g.tail_cols, g.tail_col0, g.bias,
                       static_cast<uint16_t *>(g.out), g.ld_out, g.accumulate, vec);
    return status_of(hipGetLastError());
}

// First output column of the split tail tiles (output columns: the segments' rows stacked; each
// segment's tiles run p-tile by p-tile with m fastest).
// The two parts of a head + tail plan over stacked rows (forward; `unit0` / `unit1` rows per
// p-tile of the 256x256 and 128x128 tiles: 256 / 128, or 128 / 64 for paired gate | up tiles):
// the first head_ptiles p-tiles in segment order, then each segment's remaining rows from row0.
// Returns the number of workgroups of the two-part launch.
int64_t head_tail_rows(GemmArgs &g, const Plan &p, const int64_t *rows, int nw, int64_t m,
                       int64_t unit0, int64_t unit1) {
    TileMap &ha = g.map[0], &tb = g.map[1];
    ha.m_tiles = (m + 255) / 256;
    tb.m_tiles = (m + 127) / 128;
    ha.tile_start[0] = tb.tile_start[0] = 0;
    int64_t left = p.head_ptiles;
    for (int i = 0; i < nw; ++i) {
        const int64_t pt = (rows[i] + unit0 - 1) / unit0;
        const int64_t take = left < pt ? left : pt;
        left -= take;
        const int64_t head_rows = take * unit0 < rows[i] ? take * unit0 : rows[i];
        ha.row0[i] = 0;
        tb.row0[i] = head_rows;
        ha.tile_start[i + 1] = ha.tile_start[i] + take * ha.m_tiles;
        tb.tile_start[i + 1] =
            tb.tile_start[i] + ((rows[i] - head_rows + unit1 - 1) / unit1) * tb.m_tiles;
    }
    g.blocks0 = ha.tile_start[nw];
    g.tail_start = int64_t(1) << 31;  // no split tiles in either part
    return g.blocks0 + tb.tile_start[nw];
}

// The same for dX over output columns: [0, 256 head_ptiles) in 256x256 tiles, the rest in
// 128x128 tiles from col0.
int64_t head_tail_cols(GemmArgs &g, const Plan &p, int64_t m) {
    TileMap &ha = g.map[0], &tb = g.map[1];
    const int64_t c0 = p.head_ptiles * 256 < g.K ? p.head_ptiles * 256 : g.K;
    ha.m_tiles = (m + 255) / 256;
    tb.m_tiles = (m + 127) / 128;
    ha.col0 = 0;
    tb.col0 = c0;
    g.blocks0 = (c0 / 256) * ha.m_tiles;
    g.tail_start = int64_t(1) << 31;
    return g.blocks0 + ((g.K - c0 + 127) / 128) * tb.m_tiles;
}

int64_t fwd_tail_col0(const Plan &p, int64_t m, const nf4_weight *ws, int nw) {
    const int64_t mt = (m + p.bm - 1) / p.bm;
    int64_t t = 0, col = 0;
    for (int i = 0; i < nw; ++i) {
        const int64_t tiles_i = ((ws[i].rows + p.bp - 1) / p.bp) * mt;
        if (p.tail_start < t + tiles_i) return col + ((p.tail_start - t) / mt) * p.bp;
        t += tiles_i;
        col += ws[i].rows;
    }
    return col;
}

int64_t dx_tail_col0(const Plan &p, int64_t m) {
    const int64_t mt = (m + p.bm - 1) / p.bm;
    return (p.tail_start / mt) * p.bp;
}

}  // namespace

extern "C" size_t nf4_linear_fwd_workspace(int64_t m, const nf4_weight *ws, int nw, int dtype) {
    (void)dtype;
    if (!ws || nw < 1 || nw > kMaxSeg || m <= 0) return 0;
    const Plan p = plan_fwd(m, ws, nw);
    if (p.splits <= 1) return 0;
    int64_t n = 0;
    for (int i = 0; i < nw; ++i) n += ws[i].rows;
    return static_cast<size_t>(p.splits) * m * (n - fwd_tail_col0(p, m, ws, nw)) * sizeof(float);
}

extern "C" size_t nf4_linear_dx_workspace(int64_t m, const nf4_weight *ws, int nw, int dtype) {
    (void)dtype;
    if (!ws || nw < 1 || nw > kMaxSeg || m <= 0) return 0;
    const Plan p = plan_dx(m, ws, nw);
    if (p.splits <= 1) return 0;
    return static_cast<size_t>(p.splits) * m * (ws[0].cols - dx_tail_col0(p, m)) * sizeof(float);
}

extern "C" int nf4_linear_fwd_tiled(const void *x, int64_t m, int64_t ldx, const nf4_weight *ws,
                                    int nw, const void *bias, const nf4_lora *loras, int nlora,
                                    void *y, int64_t ldy, int dtype, void *workspace,
                                    size_t workspace_bytes, void *stream, int tile, int splits) {
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
    g.act_cols = g.K;
    int xa_rank = 0;  // adapters whose down-projection T = x A^T this call computes
    for (int i = 0; i < nlora; ++i) {
        const nf4_lora &l = loras[i];
        if (l.seg < 0 || l.seg >= nw || l.rank < 1 || l.rank > 64 || !l.t || !l.b) return NF4_ERR_ARG;
        if (l.a && !aligned(l.a, 16)) return NF4_ERR_ARG;
        LoraDev &d = g.lora[l.seg];
        if (d.has) return NF4_ERR_ARG;
        d.t = static_cast<const uint16_t *>(l.t);
        d.b = static_cast<const uint16_t *>(l.b);
        d.rank = l.rank;
        d.scale = l.scale;
        d.has = 1;
        d.vec = l.rank % 8 == 0 && aligned(l.t, 16) && aligned(l.b, 16);
        if (l.a) xa_rank = l.rank > xa_rank ? l.rank : xa_rank;
    }
    if (m == 0 || n_out == 0) return NF4_OK;
    g.bias = static_cast<const uint16_t *>(bias);
    g.out = y;
    g.ld_out = ldy;
    g.n_out = n_out;
    g.vec_out = aligned(y, 8) && ldy % 4 == 0;
    g.vec16_out = aligned(y, 16) && ldy % 8 == 0;
    for (int i = 0; i < nw; ++i) {
        g.vec_out = g.vec_out && (g.seg_off[i] % 4 == 0);
        g.vec16_out = g.vec16_out && (g.seg_off[i] % 8 == 0);
    }
    bool lora_aligned = true;
    for (int i = 0; i < nlora; ++i)
        lora_aligned = lora_aligned && aligned(loras[i].b, 4) && aligned(loras[i].t, 4);
    Plan p = plan_fwd(m, ws, nw, tile, splits, lora_aligned, xa_rank);
    if (p.splits == 0) return NF4_ERR_ARG;
    if (xa_rank > 0) {
        hipStream_t s = static_cast<hipStream_t>(stream);
        p.fx = skinny_fx_ok(p, xa_rank);
        nf4_lora_job jobs[kMaxSeg];
        int nj = 0, rank0 = 0;
        bool one_rank = true;
        for (int i = 0; i < nlora; ++i) {
            const nf4_lora &l = loras[i];
            if (!l.a) continue;
            if (p.fx) {  // the skinny kernel computes T itself and writes it to t
                LoraDev &d = g.lora[l.seg];
                d.xa = static_cast<const uint16_t *>(l.a);
                d.t_out = static_cast<uint16_t *>(const_cast<void *>(l.t));
            } else {     // a launch of their own first
                jobs[nj++] = nf4_lora_job{x, ldx, g.K, l.a, const_cast<void *>(l.t), 1.0f, 0};
                one_rank = one_rank && (rank0 == 0 || rank0 == l.rank);
                rank0 = l.rank;
            }
        }
        if (nj > 0 && one_rank && nj <= NF4_MAX_LORA_JOBS) {
            st = nf4_lora_xa_multi(jobs, nj, m, rank0, dtype, s);
            if (st != NF4_OK) return st;
        } else {
            for (int i = 0; i < nlora; ++i) {
                const nf4_lora &l = loras[i];
                if (!l.a || p.fx) continue;
                st = nf4_lora_xa(x, m, g.K, ldx, l.a, l.rank, const_cast<void *>(l.t), dtype, s);
                if (st != NF4_OK) return st;
            }
        }
    }
    if (p.cfg == 6) {  // row streaming: row groups per segment, K parts per row
        g.splits = 1;
        g.rows_groups = p.rows_g;
        g.rows_parts = p.splits;
        g.map[0].tile_start[0] = 0;
        for (int i = 0; i < nw; ++i)
            g.map[0].tile_start[i + 1] =
                g.map[0].tile_start[i] +
                ((ws[i].rows + p.waves - 1) / p.waves + p.rows_g - 1) / p.rows_g * p.rows_g;
        const dim3 grid(static_cast<unsigned>(p.tiles / p.rows_g));
        const dim3 block(p.rows_g * p.splits * 64);
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (dtype == NF4_BF16) {
            if (p.bm == 1 && p.bp == 1) hipLaunchKernelGGL((gemv_rows_kernel<NF4_BF16, 1, 1>), grid, block, 0, s, g);
            else if (p.bm == 1) hipLaunchKernelGGL((gemv_rows_kernel<NF4_BF16, 1, 2>), grid, block, 0, s, g);
            else if (p.bp == 1) hipLaunchKernelGGL((gemv_rows_kernel<NF4_BF16, 2, 1>), grid, block, 0, s, g);
            else hipLaunchKernelGGL((gemv_rows_kernel<NF4_BF16, 2, 2>), grid, block, 0, s, g);
        } else {
            if (p.bm == 1 && p.bp == 1) hipLaunchKernelGGL((gemv_rows_kernel<NF4_F16, 1, 1>), grid, block, 0, s, g);
            else if (p.bm == 1) hipLaunchKernelGGL((gemv_rows_kernel<NF4_F16, 1, 2>), grid, block, 0, s, g);
            else if (p.bp == 1) hipLaunchKernelGGL((gemv_rows_kernel<NF4_F16, 2, 1>), grid, block, 0, s, g);
            else hipLaunchKernelGGL((gemv_rows_kernel<NF4_F16, 2, 2>), grid, block, 0, s, g);
        }
        return status_of(hipGetLastError());
    }
    g.splits = p.splits;
    // reduction steps per split: BR-deep steps, or the skinny path's super-steps
    const int64_t unit = p.cfg == 7 ? p.dks : BR;
    g.per_split = (g.K / unit + p.splits - 1) / p.splits;
    const int64_t bp = p.bp, bm = p.bm;
    g.map[0].m_tiles = (m + bm - 1) / bm;
    g.map[0].tile_start[0] = 0;
    for (int i = 0; i < nw; ++i)
        g.map[0].tile_start[i + 1] =
            g.map[0].tile_start[i] + ((ws[i].rows + bp - 1) / bp) * g.map[0].m_tiles;
    hipStream_t s = static_cast<hipStream_t>(stream);
    g.tail_start = p.tail_start;
    g.tail_col0 = p.splits > 1 ? fwd_tail_col0(p, m, ws, nw) : n_out;
    g.tail_cols = n_out - g.tail_col0;
    if (p.splits > 1) {
        const size_t need = static_cast<size_t>(p.splits) * m * g.tail_cols * sizeof(float);
        if (!workspace || workspace_bytes < need) return NF4_ERR_WORKSPACE;
        g.partial = static_cast<float *>(workspace);
    }
    if (p.head_ptiles > 0) {
        int64_t rows[kMaxSeg];
        for (int i = 0; i < nw; ++i) rows[i] = ws[i].rows;
        const dim3 grid(static_cast<unsigned>(head_tail_rows(g, p, rows, nw, m, 256, 128)));
        if (dtype == NF4_BF16)
            hipLaunchKernelGGL((fwd_head_tail_kernel<NF4_BF16, 0>), grid, dim3(512), 0, s, g);
        else
            hipLaunchKernelGGL((fwd_head_tail_kernel<NF4_F16, 0>), grid, dim3(512), 0, s, g);
        return status_of(hipGetLastError());
    }
    st = dtype == NF4_BF16 ? launch_fwd<NF4_BF16>(g, p, s) : launch_fwd<NF4_F16>(g, p, s);
    if (st != NF4_OK || p.splits <= 1) return st;
    return dtype == NF4_BF16 ? launch_reduce<NF4_BF16>(g, p.splits, s)
                             : launch_reduce<NF4_F16>(g, p.splits, s);
}

extern "C" int nf4_linear_fwd(const void *x, int64_t m, int64_t ldx, const nf4_weight *ws, int nw,
                              const void *bias, const nf4_lora *loras, int nlora, void *y,
                              int64_t ldy, int dtype, void *workspace, size_t workspace_bytes,
                              void *stream) {
    return nf4_linear_fwd_tiled(x, m, ldx, ws, nw, bias, loras, nlora, y, ldy, dtype, workspace,
                                workspace_bytes, stream, NF4_TILE_AUTO, 1);
}

namespace {

// nf4_linear_dx_tiled with the automatic plan restricted to split-K partials of at most
// ws_cap bytes (ws_cap < 0: no restriction).
int linear_dx_impl(const void *dy, int64_t m, int64_t lddy, const nf4_weight *ws, int nw,
                   const nf4_lora *loras, int nlora, void *dx, int64_t lddx, int accumulate,
                   int dtype, void *workspace, size_t workspace_bytes, void *stream, int tile,
                   int splits, int64_t ws_cap) {
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
    g.act_cols = n_in;
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
        d.vec = l.rank % 8 == 0 && aligned(l.da, 16);
    }
    if (m == 0 || g.K == 0) return NF4_OK;
    g.out = dx;
    g.ld_out = lddx;
    g.n_out = g.K;
    g.accumulate = accumulate != 0;
    g.vec_out = aligned(dx, 8) && lddx % 4 == 0;
    g.vec16_out = aligned(dx, 16) && lddx % 8 == 0;
    const Plan p = plan_dx(m, ws, nw, tile, splits, ws_cap);
    if (p.splits == 0) return NF4_ERR_ARG;
    g.splits = p.splits;
    const int64_t bp = p.bp, bm = p.bm;
    g.map[0].m_tiles = (m + bm - 1) / bm;
    g.step_start[0] = 0;
    for (int i = 0; i < nw; ++i) g.step_start[i + 1] = g.step_start[i] + (ws[i].rows + BR - 1) / BR;
    g.total_steps = g.step_start[nw];
    g.per_split = (g.total_steps + p.splits - 1) / p.splits;
    hipStream_t s = static_cast<hipStream_t>(stream);
    g.tail_start = p.tail_start;
    g.tail_col0 = p.splits > 1 ? dx_tail_col0(p, m) : g.K;
    g.tail_cols = g.K - g.tail_col0;
    if (p.splits > 1) {
        const size_t need = static_cast<size_t>(p.splits) * m * g.tail_cols * sizeof(float);
        if (!workspace || workspace_bytes < need) return NF4_ERR_WORKSPACE;
        g.partial = static_cast<float *>(workspace);
    }
    if (p.head_ptiles > 0) {
        const dim3 grid(static_cast<unsigned>(head_tail_cols(g, p, m)));
        if (dtype == NF4_BF16)
            hipLaunchKernelGGL((dx_head_tail_kernel<NF4_BF16>), grid, dim3(512), 0, s, g);
        else
            hipLaunchKernelGGL((dx_head_tail_kernel<NF4_F16>), grid, dim3(512), 0, s, g);
        return status_of(hipGetLastError());
    }
    st = dtype == NF4_BF16 ? launch_dx<NF4_BF16>(g, p, s) : launch_dx<NF4_F16>(g, p, s);
    if (st != NF4_OK || p.splits <= 1) return st;
    return dtype == NF4_BF16 ? launch_reduce<NF4_BF16>(g, p.splits, s)
                             : launch_reduce<NF4_F16>(g, p.splits, s);
}

// ------------------------------------------------- the allocation-free input gradient
//
// nf4_linear_dx_noalloc keeps its split-K partials in `scratch`, one array of
// NF4_STATIC_SCRATCH_BYTES per GPU, allocated when the library's code is loaded on a device
// and held until the process ends.  In host code `scratch` names a host-side stand-in, not
// device memory: its device address is looked up once per device (hipGetSymbolAddress, with
// that device current, on the entry point's first call there) and only that address is used.
// Every split tile writes all of its partials before the reduction reads them, so nothing in
// the array needs clearing between calls.  Calls that overlap on one GPU (two streams, two
// threads) share the array and race.

static __device__ __align__(256) uint8_t scratch[NF4_STATIC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxScratchDevices] = {};

// The device address of `scratch` on the current device.
int scratch_on_current_device(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return NF4_ERR_LAUNCH;
    if (dev < 0 || dev >= kMaxScratchDevices) return NF4_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p)
            return NF4_ERR_LAUNCH;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return NF4_OK;
}

}  // namespace

extern "C" int nf4_linear_dx_tiled(const void *dy, int64_t m, int64_t lddy, const nf4_weight *ws,
                                   int nw, const nf4_lora *loras, int nlora, void *dx,
                                   int64_t lddx, int accumulate, int dtype, void *workspace,
                                   size_t workspace_bytes, void *stream, int tile, int splits) {
    return linear_dx_impl(dy, m, lddy, ws, nw, loras, nlora, dx, lddx, accumulate, dtype,
                          workspace, workspace_bytes, stream, tile, splits, -1);
}

extern "C" int nf4_linear_dx(const void *dy, int64_t m, int64_t lddy, const nf4_weight *ws, int nw,
                             const nf4_lora *loras, int nlora, void *dx, int64_t lddx,
                             int accumulate, int dtype, void *workspace, size_t workspace_bytes,
                             void *stream) {
    return linear_dx_impl(dy, m, lddy, ws, nw, loras, nlora, dx, lddx, accumulate, dtype,
                          workspace, workspace_bytes, stream, NF4_TILE_AUTO, 1, -1);
}

extern "C" int nf4_linear_dx_noalloc(const void *dy, int64_t m, int64_t lddy, const nf4_weight *ws,
                                     int nw, const nf4_lora *loras, int nlora, void *dx,
                                     int64_t lddx, int accumulate, int dtype, void *stream) {
    void *ws_dev = nullptr;
    const int st = scratch_on_current_device(&ws_dev);
    if (st != NF4_OK) return st;
    // plans needing more than the array are never chosen; linear_dx_impl still checks the
    // chosen plan's need against the size passed (NF4_ERR_WORKSPACE)
    return linear_dx_impl(dy, m, lddy, ws, nw, loras, nlora, dx, lddx, accumulate, dtype, ws_dev,
                          NF4_STATIC_SCRATCH_BYTES, stream, NF4_TILE_AUTO, 1,
                          static_cast<int64_t>(NF4_STATIC_SCRATCH_BYTES));
}

namespace {

// The gate | up pair with the SwiGLU epilogue (forward: out = H [M, I]; backward: aux = dH,
// out = dG | dU [M, 2I]).  Tiles of the 256x256 or 128x128 forward kernel, chosen by the same
// cost model over the stacked 2I rows, never split (the epilogue needs whole sums).
int paired_swiglu(const void *x, int64_t m, int64_t ldx, const nf4_weight *gate_up, void *out,
                  int64_t ldo, const void *aux, int64_t ld_aux, int dtype, bool bwd, void *stream,
                  int tile = NF4_TILE_AUTO) {
    if (dtype != NF4_F16 && dtype != NF4_BF16) return NF4_ERR_ARG;
    if (m < 0 || !out || (m > 0 && !x) || (bwd && m > 0 && !aux)) return NF4_ERR_ARG;
    GemmArgs g;
    int st = fill_common(g, x, m, ldx, gate_up, 2);
    if (st != NF4_OK) return st;
    const int64_t inter = gate_up[0].rows;
    if (gate_up[1].rows != inter) return NF4_ERR_ARG;
    if (ldo < (bwd ? 2 * inter : inter) || (bwd && ld_aux < inter)) return NF4_ERR_ARG;
    if (m == 0 || inter == 0) return NF4_OK;
    g.act_cols = g.K;
    g.out = out;
    g.ld_out = ldo;
    g.n_out = bwd ? 2 * inter : inter;
    g.aux = static_cast<const uint16_t *>(aux);
    g.ld_aux = ld_aux;
    g.vec_out = aligned(out, 8) && ldo % 4 == 0 &&
                (!bwd || (inter % 4 == 0 && aligned(aux, 8) && ld_aux % 4 == 0));
    const int64_t big = ((inter + 127) / 128) * ((m + 255) / 256);
    const int64_t small = ((inter + 63) / 64) * ((m + 127) / 128);
    const Plan p = tile < 0 ? make_plan(m, big, small, g.K / BR, 1)
                            : pinned_plan(tile, 1, big, small, g.K / BR);
    if (p.splits == 0) return NF4_ERR_ARG;
    g.splits = 1;
    g.per_split = g.K / BR;
    g.map[0].m_tiles = (m + p.bm - 1) / p.bm;
    g.map[0].tile_start[0] = 0;
    g.map[0].tile_start[1] = p.tiles;
    g.tail_start = p.tiles;
    g.tail_col0 = g.n_out;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (p.head_ptiles > 0) {
        const dim3 grid(static_cast<unsigned>(head_tail_rows(g, p, &inter, 1, m, 128, 64)));
        if (dtype == NF4_BF16) {
            if (bwd) hipLaunchKernelGGL((fwd_head_tail_kernel<NF4_BF16, 2>), grid, dim3(512), 0, s, g);
            else hipLaunchKernelGGL((fwd_head_tail_kernel<NF4_BF16, 1>), grid, dim3(512), 0, s, g);
        } else {
            if (bwd) hipLaunchKernelGGL((fwd_head_tail_kernel<NF4_F16, 2>), grid, dim3(512), 0, s, g);
            else hipLaunchKernelGGL((fwd_head_tail_kernel<NF4_F16, 1>), grid, dim3(512), 0, s, g);
        }
        return status_of(hipGetLastError());
    }
    if (dtype == NF4_BF16)
        return bwd ? launch_paired<NF4_BF16, 2>(g, p, s) : launch_paired<NF4_BF16, 1>(g, p, s);
    return bwd ? launch_paired<NF4_F16, 2>(g, p, s) : launch_paired<NF4_F16, 1>(g, p, s);
}

}  // namespace

extern "C" int nf4_linear_swiglu_fwd(const void *x, int64_t m, int64_t ldx,
                                     const nf4_weight *gate_up, void *h, int64_t ldh, int dtype,
                                     void *stream) {
    return paired_swiglu(x, m, ldx, gate_up, h, ldh, nullptr, 0, dtype, false, stream);
}

extern "C" int nf4_linear_swiglu_bwd(const void *x, int64_t m, int64_t ldx,
                                     const nf4_weight *gate_up, const void *dh, int64_t lddh,
                                     void *dgu, int64_t lddgu, int dtype, void *stream) {
    return paired_swiglu(x, m, ldx, gate_up, dgu, lddgu, dh, lddh, dtype, true, stream);
}

extern "C" int nf4_linear_swiglu_tiled(const void *x, int64_t m, int64_t ldx,
                                       const nf4_weight *gate_up, void *out, int64_t ldo,
                                       const void *dh, int64_t lddh, int dtype, void *stream,
                                       int backward, int tile) {
    return paired_swiglu(x, m, ldx, gate_up, out, ldo, dh, lddh, dtype, backward != 0, stream,
                         tile);
}
