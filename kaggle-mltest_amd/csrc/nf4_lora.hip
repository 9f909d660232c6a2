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
__device__ __forceinline__ float bits_f32(uint32_t v) {  // low 16 bits of v
    if constexpr (DT == NF4_BF16) return __uint_as_float(v << 16);
    else return static_cast<float>(__builtin_bit_cast(half_t, static_cast<uint16_t>(v)));
}

template <int DT>
__device__ __forceinline__ uint16_t st1(float v) {
    return round16<DT>(v);
}

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

// 8 16-bit values src[j * stride], j < lim (the rest zero), as an MFMA fragment; one 16-byte
// load when the 8 are contiguous, in range and aligned.
__device__ __forceinline__ u32x4_t frag8(const uint16_t *src, int64_t stride, int lim, bool vec) {
    if (vec && stride == 1 && lim >= 8) return *reinterpret_cast<const u32x4_t *>(src);
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

constexpr int kMaxRank = 64;

// ds_read_b64_tr_b16: in each 16-lane group lane q points at 4 consecutive 16-bit columns of
// row r0 + q / 4 of a row-major LDS tile and receives column q of rows r0 .. r0 + 3.
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

__device__ __forceinline__ uint2 tr_read(const uint8_t *s, int off) {
    const v4i16_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4i16_t *)((__attribute__((address_space(3))) uint8_t *)s + off));
    return __builtin_bit_cast(uint2, v);
}

// One LoRA side product of a launch (the C ABI's nf4_lora_job plus host-computed layout).
struct Job {
    const uint16_t *in;   // rowdot: act rows; wgrad: U rows (already at their column offset)
    int64_t ld;
    int64_t cols;         // rowdot: reduction length; wgrad: P
    const uint16_t *w;    // rowdot: A [rank, cols] or B [cols, rank]; wgrad: V [M, rank]
    void *out;
    float scale;
    int transpose;        // wgrad: out is [rank, P]
    int vec;              // rowdot: bit 0 act rows 16-byte loadable, bit 1 A rows, bit 2 B rows;
                          // wgrad: U rows
    int64_t part_off;     // wgrad: float offset of this job's partials in the workspace
    int64_t out_start;    // wgrad: first output element of this job in the final grid
    int64_t tile0;        // one-pass wgrad: first workgroup of this job
};

struct Jobs {
    Job j[NF4_MAX_LORA_JOBS];
    int n;
};

// out[m][j] = scale * sum_k act[m][k] * W(j, k) on v_mfma_f32_16x16x32, where
//   W(j, k) = w[j * K + k]    (B_LAYOUT false: LoRA A [rank, K], for t = xd A^T)
//   W(j, k) = w[k * rank + j] (B_LAYOUT true:  LoRA B [N, rank], for da = s dY B).
// A workgroup owns 16 rows m; its 16 waves split the reduction (short per-wave ranges keep
// many loads in flight, also when M is a handful of tokens) and add their 16 x 16 partial tiles
// through LDS in a fixed order.  MFMA A operand = W (rows j), B operand = act (cols m).  In the
// B layout a 32-deep slice of B (32 rows of 16 ranks, 16-byte loads) goes through the wave's
// own LDS tile and comes back transposed (tr_read) as the A fragments, in place of 8 strided
// 2-byte loads per fragment.
constexpr int kRowdotWaves = 16;

template <int DT, bool B_LAYOUT, bool BV = false>
__global__ __launch_bounds__(kRowdotWaves * 64) void rowdot_kernel(const Jobs jobs, int64_t m,
                                                                     int rank) {
    static_assert(!BV || B_LAYOUT, "B rows through LDS in the B layout only");
    __shared__ float4_t red[kRowdotWaves][64];
    __shared__ __attribute__((aligned(16))) uint8_t sB[BV ? kRowdotWaves : 1][32 * 32];
    const Job &jb = jobs.j[blockIdx.y];
    const rsrc_t brs = make_rsrc(jb.w, BV ? jb.cols * rank * 2 : 0);  // BV: every job's B rows 16-byte loadable
    const uint16_t *act = jb.in, *w = jb.w;
    const int64_t k = jb.cols, ld = jb.ld;
    uint16_t *out = static_cast<uint16_t *>(jb.out);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t m0 = static_cast<int64_t>(blockIdx.x) * 16;
    // per-wave share of k, a multiple of 32
    const int64_t kc = ((k + 32 * kRowdotWaves - 1) / (32 * kRowdotWaves)) * 32;
    const int64_t kb = wave * kc;
    const int64_t ke = kb + kc < k ? kb + kc : k;
    const int col = lane & 15, kq = (lane >> 4) * 8;
    const int64_t row = m0 + col;
    for (int j0 = 0; j0 < rank; j0 += 16) {
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
        const int j = j0 + col;
        // U 32-deep slices per group: all their loads are issued before the first MFMA, so a
        // wave waits for one memory latency per group, not per slice
        constexpr int kRowdotUnroll = B_LAYOUT && !BV ? 2 : B_LAYOUT ? 4 : 8;
        for (int64_t k0 = kb; k0 < ke; k0 += 32 * kRowdotUnroll) {
            u32x4_t fa[kRowdotUnroll], fb[kRowdotUnroll], rb[BV ? kRowdotUnroll : 1];
#pragma unroll
            for (int u = 0; u < kRowdotUnroll; ++u) {
                const int64_t kk = k0 + 32 * u + kq;
                const int lim = ke - kk < 8 ? static_cast<int>(ke - kk) : 8;
                fa[u] = (u32x4_t){0u, 0u, 0u, 0u};
                fb[u] = (u32x4_t){0u, 0u, 0u, 0u};
                if constexpr (BV) {
                    // rows k0 + 32 u + lane / 2 of B, ranks j0 + 8 (lane % 2) ..: rows past K
                    // read as zero, rows past the wave's range meet zero activations, ranks
                    // past the rank reach outputs that are not stored
                    rb[u] = bload16(brs, static_cast<int>(((k0 + 32 * u + (lane >> 1)) * rank +
                                                           j0 + (lane & 1) * 8) * 2));
                } else if (lim > 0 && j < rank) {
                    fa[u] = B_LAYOUT ? frag8(w + kk * rank + j, rank, lim, false)
                                     : frag8(w + j * k + kk, 1, lim, (jb.vec & 2) != 0);
                }
                if (lim > 0 && row < m) fb[u] = frag8(act + row * ld + kk, 1, lim, (jb.vec & 1) != 0);
            }
            if constexpr (BV) {
                uint8_t *sb = sB[wave];
                const int r0 = 8 * (lane >> 4) + ((lane & 15) >> 2), c4 = (lane & 3) * 8;
#pragma unroll
                for (int u = 0; u < kRowdotUnroll; ++u) {
                    *reinterpret_cast<u32x4_t *>(sb + (lane >> 1) * 32 + (lane & 1) * 16) = rb[u];
                    const uint2 lo = tr_read(sb, r0 * 32 + c4), hi = tr_read(sb, (r0 + 4) * 32 + c4);
                    fa[u] = (u32x4_t){lo.x, lo.y, hi.x, hi.y};
                }
            }
#pragma unroll
            for (int u = 0; u < kRowdotUnroll; ++u) acc = mfma16<DT>(fa[u], fb[u], acc);
        }
        red[wave][lane] = acc;
        __syncthreads();
        if (wave == 0) {
            float4_t s = red[0][lane];
            for (int v = 1; v < kRowdotWaves; ++v) s += red[v][lane];
            const int64_t mm = m0 + (lane & 15);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int jj = j0 + (lane >> 4) * 4 + q;
                if (mm < m && jj < rank) out[mm * rank + jj] = st1<DT>(s[q] * jb.scale);
            }
        }
        __syncthreads();
    }
}

// Decode-size xa (M <= kRowvecMaxM tokens): out[m][j] = scale * sum_k act[m][k] A[j][k] with one
// workgroup per (job, row j of A, group of MT tokens) over the whole reduction, instead of one
// workgroup per 16 tokens and job: each of 256 threads takes 8 consecutive k per 2048-wide step
// (16-byte loads of the A row and of every token's activations), accumulates with v_dot2 in
// fp32, and the workgroup adds its lanes in a fixed order (DPP inside each wave, then the four
// waves in order).  The MFMA kernel above streams A and 16 tokens through a single CU per 16
// tokens (K = 3584: 8.2 us for 16 tokens, whatever M up to 64); here the rank x token-group
// workgroups spread them over the GPU.  Needs 16-byte aligned rows (Job::vec == 3).
constexpr int64_t kRowvecMaxM = 64;

template <int DT, int MT>
__global__ __launch_bounds__(256) void rowvec_kernel(const Jobs jobs, int64_t m_all) {
    __shared__ float red[4][MT];
    const Job &jb = jobs.j[blockIdx.y];
    const int64_t k = jb.cols, ld = jb.ld;
    const int rank = static_cast<int>(gridDim.x);
    const int j = blockIdx.x;
    const int64_t t0 = static_cast<int64_t>(blockIdx.z) * MT;  // this workgroup's first token
    const int64_t m = m_all - t0 < MT ? m_all - t0 : MT;
    const uint16_t *w = jb.w + j * k;
    const uint16_t *in = jb.in + t0 * ld;
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
#pragma unroll 2
    for (int64_t k0 = threadIdx.x * 8; k0 < k; k0 += 256 * 8) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t *>(w + k0);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t >= m) break;
            const u32x4_t x = *reinterpret_cast<const u32x4_t *>(in + t * ld + k0);
            acc[t] = dot2<DT>(a.w, x.w, dot2<DT>(a.z, x.z, dot2<DT>(a.y, x.y, dot2<DT>(a.x, x.x, acc[t]))));
        }
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const float v = wave_sum(acc[t]);
        if (lane == 0) red[wave][t] = v;
    }
    __syncthreads();
    if (threadIdx.x < MT && threadIdx.x < m) {
        const int t = threadIdx.x;
        const float v = ((red[0][t] + red[1][t]) + red[2][t]) + red[3][t];
        static_cast<uint16_t *>(jb.out)[(t0 + t) * rank + j] = st1<DT>(v * jb.scale);
    }
}

// The LoRA term of the input gradient, unfolded (the dropout-masked branch of the norm
// backward needs it on its own): out[m][k] = scale * sum_j da[m][j] A[j][k] for a job with
// in = da [M, rank] (row stride ld), w = A [rank, cols], out [M, cols] contiguous.  A thread
// owns one column k (A's column in registers) over a block of kAxRows rows whose da rows are
// staged in LDS; fp32 sums over j in order, rounded once.  Bound by the output's writes.
constexpr int kAxRows = 16;

template <int DT>
__global__ __launch_bounds__(256) void lora_ax_kernel(const Jobs jobs, int64_t m, int rank) {
    __shared__ float s_da[kAxRows][kMaxRank];
    const Job &jb = jobs.j[blockIdx.z];
    const int64_t k = jb.cols;
    const int64_t col = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kAxRows;
    for (int i = threadIdx.x; i < kAxRows * rank; i += 256) {
        const int r = i / rank, j = i - r * rank;
        s_da[r][j] = m0 + r < m ? ld1<DT>(jb.in + (m0 + r) * jb.ld + j) : 0.0f;
    }
    float a[kMaxRank];
#pragma unroll
    for (int j = 0; j < kMaxRank; ++j) a[j] = (j < rank && col < k) ? ld1<DT>(jb.w + j * k + col) : 0.0f;
    __syncthreads();
    if (col >= k) return;
    uint16_t *out = static_cast<uint16_t *>(jb.out);
    for (int r = 0; r < kAxRows; ++r) {
        if (m0 + r >= m) break;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxRank; ++j)
            if (j < rank) acc += s_da[r][j] * a[j];
        out[(m0 + r) * k + col] = st1<DT>(acc * jb.scale);
    }
}

// Partial sums over a chunk of rows on v_mfma_f32_16x16x32:
//   part[chunk][p][j] = sum_{m in chunk} U[m][p] * V[m][j]
// for a 64-column tile of p (4 waves x 16) and one 16-wide tile of j (blockIdx.z).  Both
// operands are reduced over m, so they are staged in LDS transposed ([p][m], [j][m]) and the
// MFMA fragments are contiguous 16-byte LDS reads.  The chunk runs in blocks of 128 rows: each
// thread issues the loads of all four 32-row slices of a block before its first LDS store, so a
// workgroup waits for one memory latency per block; the slices then go through the MFMA in
// order (the same sums in the same order as one slice at a time).  LDS rows of 136 halves
// (272 bytes, 17 chunks): the 16 rows of a fragment read start on 16 different bank groups.
// Grid: x = 64-column p tiles (of the widest job), y = row chunks, z = job x 16-wide j tiles.
template <int DT>
__global__ __launch_bounds__(256) void wgrad_partial_kernel(const Jobs jobs, int64_t m, int rank,
                                                            int64_t rows_per_chunk, float *ws) {
    constexpr int MB = 128;     // rows of a block
    constexpr int SR = MB + 8;  // LDS row (halves)
    __shared__ __attribute__((aligned(16))) uint16_t sU[64 * SR];
    __shared__ __attribute__((aligned(16))) uint16_t sV[16 * SR];
    const int jtiles = (rank + 15) / 16;
    const Job &jb = jobs.j[blockIdx.z / jtiles];
    const uint16_t *u = jb.in, *v = jb.w;
    const int64_t p = jb.cols, ldu = jb.ld;
    const bool vec_u = jb.vec != 0;
    float *part = ws + jb.part_off;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t p0 = static_cast<int64_t>(blockIdx.x) * 64;
    if (p0 >= p) return;  // a narrower job than the grid (uniform per workgroup)
    const int64_t chunk = blockIdx.y;
    const int j0 = (blockIdx.z % jtiles) * 16;
    const int64_t r0 = chunk * rows_per_chunk;
    const int64_t r1 = r0 + rows_per_chunk < m ? r0 + rows_per_chunk : m;
    // U: thread -> 8 columns pc .. pc + 7 of rows ur + 32 s; V: 8 of the 16 j of row vr
    const int ur = threadIdx.x >> 3, pc = (threadIdx.x & 7) * 8;
    const int vr = threadIdx.x >> 1, jc = (threadIdx.x & 1) * 8;
    const int ulim = p - (p0 + pc) < 8 ? static_cast<int>(p - (p0 + pc)) : 8;
    const int vlim = rank - (j0 + jc) < 8 ? rank - (j0 + jc) : 8;
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int64_t mb = r0; mb < r1; mb += MB) {
        u32x4_t xu[MB / 32], xv = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int sl = 0; sl < MB / 32; ++sl) {
            const int64_t mm = mb + 32 * sl + ur;
            xu[sl] = (mm < r1 && ulim > 0) ? frag8(u + mm * ldu + p0 + pc, 1, ulim, vec_u)
                                           : (u32x4_t){0u, 0u, 0u, 0u};
        }
        if (mb + vr < r1 && vlim > 0) xv = frag8(v + (mb + vr) * rank + j0 + jc, 1, vlim, false);
        if (mb > r0) __syncthreads();  // the previous block's fragment reads are done
#pragma unroll
        for (int sl = 0; sl < MB / 32; ++sl) {
            const uint32_t xw[4] = {xu[sl].x, xu[sl].y, xu[sl].z, xu[sl].w};
#pragma unroll
            for (int q = 0; q < 8; ++q)
                sU[(pc + q) * SR + 32 * sl + ur] = static_cast<uint16_t>(xw[q >> 1] >> ((q & 1) * 16));
        }
        {
            const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (int q = 0; q < 8; ++q)
                sV[(jc + q) * SR + vr] = static_cast<uint16_t>(xw[q >> 1] >> ((q & 1) * 16));
        }
        __syncthreads();
#pragma unroll
        for (int sl = 0; sl < MB / 32; ++sl) {
            const int off = 32 * sl + (lane >> 4) * 8;
            const u32x4_t fa =
                *reinterpret_cast<const u32x4_t *>(sU + (wave * 16 + (lane & 15)) * SR + off);
            const u32x4_t fb = *reinterpret_cast<const u32x4_t *>(sV + (lane & 15) * SR + off);
            acc = mfma16<DT>(fa, fb, acc);
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t pp = p0 + wave * 16 + (lane >> 4) * 4 + q;
        const int jj = j0 + (lane & 15);
        if (pp < p && jj < rank) part[(chunk * p + pp) * rank + jj] = acc[q];
    }
}

// out = scale * sum over chunks of part[chunk][p][j] ([p, rank], or [rank, p] transposed), for
// every job: the grid covers all jobs' outputs back to back.  Thread i owns output element i of
// its job's stored layout (coalesced stores); four independent partial sums over chunks
// c = 0, 1, 2, 3 mod 4 keep four loads in flight and are added in a fixed order (deterministic).
__global__ __launch_bounds__(256) void wgrad_final_kernel(const Jobs jobs, const float *ws,
                                                          int chunks, int rank, int64_t total) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (g >= total) return;
    int ji = 0;
#pragma unroll
    for (int q = 1; q < NF4_MAX_LORA_JOBS; ++q)
        if (q < jobs.n && g >= jobs.j[q].out_start) ji = q;
    const Job &jb = jobs.j[ji];
    const float *part = ws + jb.part_off;
    const int64_t p = jb.cols;
    const int64_t i = g - jb.out_start;
    // 32-bit index arithmetic (p * rank < 2^31 is checked on the host)
    const uint32_t ui = static_cast<uint32_t>(i), up = static_cast<uint32_t>(p);
    const int64_t src = jb.transpose ? static_cast<int64_t>(ui % up) * rank + ui / up : i;
    const int64_t stride = p * rank;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    int c = 0;
    for (; c + 4 <= chunks; c += 4) {
#pragma unroll
        for (int q = 0; q < 4; ++q) s[q] += part[(c + q) * stride + src];
    }
    for (int q = 0; c < chunks; ++c, ++q) s[q] += part[c * stride + src];
    static_cast<float *>(jb.out)[i] = ((s[0] + s[1]) + (s[2] + s[3])) * jb.scale;
}

// The weight gradients in one pass over M, for operands whose rows load as 16-byte pieces
// (U rows 16-byte aligned with ld % 8 == 0, V = [M, rank] with rank % 8 == 0):
//   out = scale * U^T V  for a 32-column tile of p and a 16-wide tile of j per workgroup.
// Wave w of the kWgWaves takes the 32-row slices w, w + kWgWaves, .. of M with kWgRing slices
// of loads in flight (buffer loads: rows past M read as zero; columns past p or rank read what
// follows in memory and only reach outputs that are not stored; 8 waves measured 7 % faster
// than 4 on the bench's layer).  A slice goes through the wave's own LDS
// tile in its natural layout ([m][p], [m][j]) and comes back transposed by
// ds_read_b64_tr_b16 as the MFMA fragments (A = U^T: 16 p x 32 m, B = V: 32 m x 16 j; in each
// 16-lane group lane q points at 4 consecutive columns of row m0 + q / 4 and receives column
// q of rows m0 .. m0 + 3).  The waves' sums are added in wave order through LDS: deterministic,
// no partials and no second launch.  Grid: the jobs' (p tile x j tile) workgroups back to back.
constexpr int kWgCols = 32;
constexpr int kWgRing = 4;
constexpr int kWgWaves = 8;
constexpr int64_t kWgPastRows = 32 * kWgWaves * 3 * kWgRing;  // rows the ring may load past M

template <int DT>
__global__ __launch_bounds__(kWgWaves * 64) void wgrad_direct_kernel(const Jobs jobs, int64_t m,
                                                                     int rank) {
    constexpr int NW = kWgWaves;
    __shared__ __attribute__((aligned(16))) uint8_t sU[NW][32 * kWgCols * 2];  // [m][p], 64 B rows
    __shared__ __attribute__((aligned(16))) uint8_t sV[NW][32 * 16 * 2];       // [m][j], 32 B rows
    __shared__ float4_t red[NW][2][64];
    int ji = 0;
#pragma unroll
    for (int q = 1; q < NF4_MAX_LORA_JOBS; ++q)
        if (q < jobs.n && static_cast<int64_t>(blockIdx.x) >= jobs.j[q].tile0) ji = q;
    const Job &jb = jobs.j[ji];
    const int jtiles = (rank + 15) / 16;
    const int lt = static_cast<int>(blockIdx.x - jb.tile0);
    const int64_t p = jb.cols;
    const int p0 = (lt / jtiles) * kWgCols, j0 = (lt % jtiles) * 16;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    // 32-bit byte offsets: the host checks (m + kWgPastRows) * ld * 2 < 2^31, which covers the
    // ring's loads past the last slice
    const rsrc_t ur = make_rsrc(jb.in, m * jb.ld * 2);
    const rsrc_t vr = make_rsrc(jb.w, m * rank * 2);
    const int row = lane >> 1, half = lane & 1;
    const int uoff = row * static_cast<int>(jb.ld) * 2 + (p0 + half * 16) * 2;
    const int voff = row * rank * 2 + (j0 + half * 8) * 2;
    const int uslice = 32 * static_cast<int>(jb.ld) * 2, vslice = 32 * rank * 2;
    const int nsl = static_cast<int>((m + 31) / 32);
    const int cnt = nsl > wave ? (nsl - wave + NW - 1) / NW : 0;
    u32x4_t ru[kWgRing][2], rv[kWgRing];
    auto load = [&](int d, int i) {  // wave slice i: rows 32 (wave + NW i) ..
        const int sl = wave + NW * i;
        ru[d][0] = bload16(ur, uoff + sl * uslice);
        ru[d][1] = bload16(ur, uoff + sl * uslice + 16);
        rv[d] = bload16(vr, voff + sl * vslice);
    };
#pragma unroll
    for (int d = 0; d < kWgRing; ++d) load(d, d);
    uint8_t *su = sU[wave], *sv = sV[wave];
    const int q = lane & 15, g = lane >> 4;
    float4_t acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    for (int i0 = 0; i0 < cnt; i0 += kWgRing) {
#pragma unroll
        for (int d = 0; d < kWgRing; ++d) {
            if (i0 + d < cnt) {
                *reinterpret_cast<u32x4_t *>(su + row * 64 + half * 32) = ru[d][0];
                *reinterpret_cast<u32x4_t *>(su + row * 64 + half * 32 + 16) = ru[d][1];
                *reinterpret_cast<u32x4_t *>(sv + row * 32 + half * 16) = rv[d];
                const int r0 = 8 * g + (q >> 2), c4 = (q & 3) * 8;  // row, byte column of 4
                const uint2 vl = tr_read(sv, r0 * 32 + c4), vh = tr_read(sv, (r0 + 4) * 32 + c4);
                const u32x4_t fb = {vl.x, vl.y, vh.x, vh.y};
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const uint2 al = tr_read(su, r0 * 64 + t * 32 + c4);
                    const uint2 ah = tr_read(su, (r0 + 4) * 64 + t * 32 + c4);
                    acc[t] = mfma16<DT>((u32x4_t){al.x, al.y, ah.x, ah.y}, fb, acc[t]);
                }
            }
            load(d, i0 + d + kWgRing);
        }
    }
    red[wave][0][lane] = acc[0];
    red[wave][1][lane] = acc[1];
    __syncthreads();
    if (wave != 0) return;
    float *out = static_cast<float *>(jb.out);
    const int jj = j0 + q;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        float4_t sum = red[0][t][lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) sum += red[w][t][lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t pp = p0 + 16 * t + 4 * g + r;
            if (pp < p && jj < rank)
                out[jb.transpose ? jj * p + pp : pp * rank + jj] = sum[r] * jb.scale;
        }
    }
}

// Grid: x = column groups of 256, y = rows (grid-stride); row-strided operands.
template <int DT>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const uint16_t *gate, const uint16_t *up,
                                                         int64_t ld_gu, uint16_t *out, int64_t ld_h,
                                                         int64_t rows, int64_t cols) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (c >= cols) return;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
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
    const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (c >= cols) return;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
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

// Column sums of dY [M, N] in one pass: a workgroup owns kColsumCols = 64 columns; thread t
// takes 8 of them (chunk t % 8: one 16-byte load per row when `vec`) and the rows r with
// r % 32 == t / 8, in increasing order, 8 rows' loads in flight; the 32 row-lane sums of a
// column are then added in row-lane order through LDS (deterministic).
constexpr int kColsumCols = 64;
template <int DT>
__global__ __launch_bounds__(256) void colsum_kernel(const uint16_t *dy, int64_t m, int64_t n,
                                                     int64_t ld, int vec, float *out) {
    __shared__ float s_part[32][kColsumCols + 1];
    const int t = threadIdx.x, cq = t & 7, rl = t >> 3;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kColsumCols + cq * 8;
    const int nc = n - c0 >= 8 ? 8 : (n - c0 > 0 ? static_cast<int>(n - c0) : 0);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t r = rl;
    if (vec && nc == 8) {
        for (; r + 7 * 32 < m; r += 8 * 32) {
            u32x4_t v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = *reinterpret_cast<const u32x4_t *>(dy + (r + u * 32) * ld + c0);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc[2 * e] += bits_f32<DT>(w[e] & 0xffff);
                    acc[2 * e + 1] += bits_f32<DT>(w[e] >> 16);
                }
            }
        }
        for (; r < m; r += 32) {
            const u32x4_t v = *reinterpret_cast<const u32x4_t *>(dy + r * ld + c0);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[2 * e] += bits_f32<DT>(w[e] & 0xffff);
                acc[2 * e + 1] += bits_f32<DT>(w[e] >> 16);
            }
        }
    } else {
        for (; r < m; r += 32)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (e < nc) acc[e] += ld1<DT>(dy + r * ld + c0 + e);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) s_part[rl][cq * 8 + e] = acc[e];
    __syncthreads();
    if (t < kColsumCols) {
        const int64_t c = static_cast<int64_t>(blockIdx.x) * kColsumCols + t;
        float sum = 0.f;
        for (int i = 0; i < 32; ++i) sum += s_part[i][t];
        if (c < n) out[c] = sum;
    }
}

__global__ __launch_bounds__(256) void zero_kernel(float *out, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        out[i] = 0.f;
}

// x: column groups of 256; y: rows, at most 4096 workgroup rows (grid-stride beyond).
dim3 grid_2d(int64_t rows, int64_t cols) {
    const int64_t x = (cols + 255) / 256;
    const int64_t y = rows < 4096 ? rows : 4096;
    return dim3(static_cast<unsigned>(x), static_cast<unsigned>(y < 1 ? 1 : y));
}

int grid_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    return static_cast<int>(b > 16384 ? 16384 : (b < 1 ? 1 : b));
}

// Rows of M per wgrad workgroup: about 512 workgroups over the (64-column p tile x chunk) grid,
// at most 32 chunks, in multiples of the 32-row step.
int64_t wgrad_rows_per_chunk(int64_t m, int64_t p) {
    const int64_t p_tiles = (p + 63) / 64;
    int64_t chunks = 512 / p_tiles;
    if (chunks > 32) chunks = 32;  // the final sum reads every chunk's partial per output
    if (chunks < 1) chunks = 1;
    int64_t rows = (m + chunks - 1) / chunks;
    rows = ((rows + 31) / 32) * 32;
    return rows < 32 ? 32 : rows;
}

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

namespace {

int check_jobs(const nf4_lora_job *jobs, int njobs, int64_t m, int rank, int dtype) {
    if ((dtype != NF4_F16 && dtype != NF4_BF16) || m < 0 || rank < 1 || rank > kMaxRank)
        return NF4_ERR_ARG;
    if (!jobs || njobs < 1 || njobs > NF4_MAX_LORA_JOBS) return NF4_ERR_ARG;
    for (int i = 0; i < njobs; ++i) {
        const nf4_lora_job &j = jobs[i];
        if (j.cols < 0 || j.ld < j.cols || !j.out) return NF4_ERR_ARG;
        if (m > 0 && j.cols > 0 && (!j.in || !j.w)) return NF4_ERR_ARG;
    }
    if ((m + 15) / 16 > 0x7fffffff) return NF4_ERR_UNSUPPORTED;
    return NF4_OK;
}

Jobs to_jobs(const nf4_lora_job *jobs, int njobs) {
    Jobs J = {};
    J.n = njobs;
    for (int i = 0; i < njobs; ++i) {
        const nf4_lora_job &j = jobs[i];
        J.j[i] = Job{static_cast<const uint16_t *>(j.in), j.ld, j.cols,
                     static_cast<const uint16_t *>(j.w), j.out, j.scale, j.transpose_out != 0, 0,
                     0, 0, 0};
    }
    return J;
}

// xa (A rows contiguous) or da (B columns strided) for every job, one launch.
template <bool B_LAYOUT>
int rowdot_multi(const nf4_lora_job *jobs, int njobs, int64_t m, int rank, int dtype,
                 void *stream) {
    int st = check_jobs(jobs, njobs, m, rank, dtype);
    if (st != NF4_OK || m == 0) return st;
    Jobs J = to_jobs(jobs, njobs);
    for (int i = 0; i < njobs; ++i) {
        Job &j = J.j[i];
        j.vec = (j.ld % 8 == 0 && aligned(j.in, 16) ? 1 : 0) |
                (!B_LAYOUT && j.cols % 8 == 0 && aligned(j.w, 16) ? 2 : 0) |
                (B_LAYOUT && rank % 8 == 0 && aligned(j.w, 16) &&
                 (j.cols + 64) * rank * 2 < (int64_t(1) << 31) ? 4 : 0);
    }
    auto s = static_cast<hipStream_t>(stream);
    bool vec = true;
    for (int i = 0; i < njobs; ++i) vec = vec && J.j[i].vec == 3;
    if (!B_LAYOUT && vec && m <= kRowvecMaxM) {
        const int mt = m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8;
        const dim3 grid(static_cast<unsigned>(rank), static_cast<unsigned>(njobs),
                        static_cast<unsigned>((m + mt - 1) / mt));
#define NF4_ROWVEC(DT, MT) hipLaunchKernelGGL((rowvec_kernel<DT, MT>), grid, dim3(256), 0, s, J, m)
        if (dtype == NF4_BF16) {
            if (mt == 1) NF4_ROWVEC(NF4_BF16, 1);
            else if (mt == 2) NF4_ROWVEC(NF4_BF16, 2);
            else if (mt == 4) NF4_ROWVEC(NF4_BF16, 4);
            else NF4_ROWVEC(NF4_BF16, 8);
        } else {
            if (mt == 1) NF4_ROWVEC(NF4_F16, 1);
            else if (mt == 2) NF4_ROWVEC(NF4_F16, 2);
            else if (mt == 4) NF4_ROWVEC(NF4_F16, 4);
            else NF4_ROWVEC(NF4_F16, 8);
        }
#undef NF4_ROWVEC
        return status_of(hipGetLastError());
    }
    const dim3 grid(static_cast<unsigned>((m + 15) / 16), static_cast<unsigned>(njobs));
    bool bv = B_LAYOUT;
    for (int i = 0; i < njobs; ++i) bv = bv && (J.j[i].vec & 4) != 0;
    if (bv) {
        if (dtype == NF4_BF16)
            hipLaunchKernelGGL((rowdot_kernel<NF4_BF16, true, true>), grid, dim3(kRowdotWaves * 64),
                               0, s, J, m, rank);
        else
            hipLaunchKernelGGL((rowdot_kernel<NF4_F16, true, true>), grid, dim3(kRowdotWaves * 64),
                               0, s, J, m, rank);
    } else if (dtype == NF4_BF16)
        hipLaunchKernelGGL((rowdot_kernel<NF4_BF16, B_LAYOUT>), grid, dim3(kRowdotWaves * 64), 0,
                           s, J, m, rank);
    else
        hipLaunchKernelGGL((rowdot_kernel<NF4_F16, B_LAYOUT>), grid, dim3(kRowdotWaves * 64), 0,
                           s, J, m, rank);
    return status_of(hipGetLastError());
}

// The one-pass wgrad kernel up to this many rows, or from this many workgroups on (fewer leave
// most CUs idle over a long M: row chunks then spread the reduction).
constexpr int64_t kWgDirectMaxRows = 4096;
constexpr int64_t kWgDirectMinTiles = 128;

// Layout of the wgrad partials: rows per chunk from the widest job, jobs back to back.
struct WgradLayout {
    int64_t rows, chunks, maxp, floats, outputs;
};

WgradLayout wgrad_layout(const nf4_lora_job *jobs, int njobs, int64_t m, int rank, Jobs *J) {
    WgradLayout L = {};
    for (int i = 0; i < njobs; ++i) L.maxp = jobs[i].cols > L.maxp ? jobs[i].cols : L.maxp;
    L.rows = wgrad_rows_per_chunk(m, L.maxp > 0 ? L.maxp : 1);
    L.chunks = (m + L.rows - 1) / L.rows;
    for (int i = 0; i < njobs; ++i) {
        if (J) {
            J->j[i].part_off = L.floats;
            J->j[i].out_start = L.outputs;
        }
        L.floats += L.chunks * jobs[i].cols * rank;
        L.outputs += jobs[i].cols * rank;
    }
    return L;
}

}  // namespace

extern "C" int nf4_lora_xa_multi(const nf4_lora_job *jobs, int njobs, int64_t m, int rank,
                                 int dtype, void *stream) {
    return rowdot_multi<false>(jobs, njobs, m, rank, dtype, stream);
}

extern "C" int nf4_lora_da_multi(const nf4_lora_job *jobs, int njobs, int64_t m, int rank,
                                 int dtype, void *stream) {
    return rowdot_multi<true>(jobs, njobs, m, rank, dtype, stream);
}

extern "C" int nf4_lora_ax_multi(const nf4_lora_job *jobs, int njobs, int64_t m, int rank,
                                 int dtype, void *stream) {
    if ((dtype != NF4_F16 && dtype != NF4_BF16) || m < 0 || rank < 1 || rank > kMaxRank)
        return NF4_ERR_ARG;
    if (!jobs || njobs < 1 || njobs > NF4_MAX_LORA_JOBS) return NF4_ERR_ARG;
    int64_t maxk = 0;
    for (int i = 0; i < njobs; ++i) {
        const nf4_lora_job &j = jobs[i];
        if (j.cols < 0 || j.ld < rank || !j.out) return NF4_ERR_ARG;
        if (m > 0 && j.cols > 0 && (!j.in || !j.w)) return NF4_ERR_ARG;
        maxk = j.cols > maxk ? j.cols : maxk;
    }
    if (m == 0 || maxk == 0) return NF4_OK;
    if ((m + kAxRows - 1) / kAxRows > 65535 || (maxk + 255) / 256 > 0x7fffffff)
        return NF4_ERR_UNSUPPORTED;
    Jobs J = to_jobs(jobs, njobs);
    const dim3 grid(static_cast<unsigned>((maxk + 255) / 256),
                    static_cast<unsigned>((m + kAxRows - 1) / kAxRows), static_cast<unsigned>(njobs));
    auto s = static_cast<hipStream_t>(stream);
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL(lora_ax_kernel<NF4_BF16>, grid, dim3(256), 0, s, J, m, rank);
    else
        hipLaunchKernelGGL(lora_ax_kernel<NF4_F16>, grid, dim3(256), 0, s, J, m, rank);
    return status_of(hipGetLastError());
}

extern "C" int nf4_lora_xa(const void *xd, int64_t m, int64_t k, int64_t ldx, const void *a,
                           int rank, void *t, int dtype, void *stream) {
    if (m > 0 && (!xd || !a || !t)) return NF4_ERR_ARG;
    const nf4_lora_job j = {xd, ldx, k, a, t, 1.0f, 0};
    return nf4_lora_xa_multi(&j, 1, m, rank, dtype, stream);
}

extern "C" int nf4_lora_da(const void *dy, int64_t m, int64_t n, int64_t lddy, const void *b,
                           int rank, float scale, void *da, int dtype, void *stream) {
    if (m > 0 && (!dy || !b || !da)) return NF4_ERR_ARG;
    const nf4_lora_job j = {dy, lddy, n, b, da, scale, 0};
    return nf4_lora_da_multi(&j, 1, m, rank, dtype, stream);
}

extern "C" size_t nf4_lora_wgrad_multi_workspace(const nf4_lora_job *jobs, int njobs, int64_t m,
                                                 int rank) {
    if (!jobs || njobs < 1 || njobs > NF4_MAX_LORA_JOBS || m <= 0 || rank <= 0) return 0;
    return static_cast<size_t>(wgrad_layout(jobs, njobs, m, rank, nullptr).floats) *
           sizeof(float);
}

extern "C" int nf4_lora_wgrad_multi(const nf4_lora_job *jobs, int njobs, int64_t m, int rank,
                                    int dtype, void *workspace, size_t workspace_bytes,
                                    void *stream) {
    int st = check_jobs(jobs, njobs, m, rank, dtype);
    if (st != NF4_OK) return st;
    auto s = static_cast<hipStream_t>(stream);
    Jobs J = to_jobs(jobs, njobs);
    const WgradLayout L = wgrad_layout(jobs, njobs, m, rank, &J);
    if (L.outputs == 0) return NF4_OK;
    for (int i = 0; i < njobs; ++i)
        if (jobs[i].cols * rank >= (int64_t(1) << 31)) return NF4_ERR_UNSUPPORTED;
    if (m == 0) {  // zero gradients, by fill kernels (no memset nodes if the call is captured)
        for (int i = 0; i < njobs; ++i) {
            const int64_t n = jobs[i].cols * rank;
            if (n == 0) continue;
            hipLaunchKernelGGL(zero_kernel, dim3(grid_for(n)), dim3(256), 0, s,
                               static_cast<float *>(jobs[i].out), n);
        }
        return status_of(hipGetLastError());
    }
    // One pass over M (no workspace) when every job's rows load as 16-byte pieces and the
    // (p tile x j tile) workgroups fill the GPU; else row chunks with partial sums and a final
    // fixed-order pass.
    {
        bool direct = rank % 8 == 0;
        int64_t tiles = 0;
        for (int i = 0; i < njobs; ++i) {
            Job &j = J.j[i];
            direct = direct && j.ld % 8 == 0 && aligned(j.in, 16) && aligned(j.w, 16) &&
                     (m + kWgPastRows) * j.ld * 2 < (int64_t(1) << 31) &&
                     (m + kWgPastRows) * rank * 2 < (int64_t(1) << 31);
            j.tile0 = tiles;
            tiles += (jobs[i].cols + kWgCols - 1) / kWgCols * ((rank + 15) / 16);
        }
        if (direct && (m <= kWgDirectMaxRows || tiles >= kWgDirectMinTiles) && tiles <= 0x7fffffff) {
            if (dtype == NF4_BF16)
                hipLaunchKernelGGL(wgrad_direct_kernel<NF4_BF16>, dim3(static_cast<unsigned>(tiles)),
                                   dim3(kWgWaves * 64), 0, s, J, m, rank);
            else
                hipLaunchKernelGGL(wgrad_direct_kernel<NF4_F16>, dim3(static_cast<unsigned>(tiles)),
                                   dim3(kWgWaves * 64), 0, s, J, m, rank);
            return status_of(hipGetLastError());
        }
    }
    const size_t need = static_cast<size_t>(L.floats) * sizeof(float);
    if (!workspace || workspace_bytes < need) return NF4_ERR_WORKSPACE;
    if (L.chunks > 65535 || static_cast<int64_t>(njobs) * ((rank + 15) / 16) > 65535)
        return NF4_ERR_UNSUPPORTED;
    for (int i = 0; i < njobs; ++i) {
        Job &j = J.j[i];
        j.vec = j.ld % 8 == 0 && aligned(j.in, 16) ? 1 : 0;
    }
    float *ws = static_cast<float *>(workspace);
    const dim3 grid(static_cast<unsigned>((L.maxp + 63) / 64), static_cast<unsigned>(L.chunks),
                    static_cast<unsigned>(njobs * ((rank + 15) / 16)));
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL(wgrad_partial_kernel<NF4_BF16>, grid, dim3(256), 0, s, J, m, rank,
                           L.rows, ws);
    else
        hipLaunchKernelGGL(wgrad_partial_kernel<NF4_F16>, grid, dim3(256), 0, s, J, m, rank,
                           L.rows, ws);
    st = status_of(hipGetLastError());
    if (st != NF4_OK) return st;
    hipLaunchKernelGGL(wgrad_final_kernel, dim3(static_cast<unsigned>((L.outputs + 255) / 256)),
                       dim3(256), 0, s, J, ws, static_cast<int>(L.chunks), rank, L.outputs);
    return status_of(hipGetLastError());
}

extern "C" size_t nf4_lora_wgrad_workspace(int64_t m, int64_t p, int rank) {
    const nf4_lora_job j = {nullptr, p, p, nullptr, nullptr, 1.0f, 0};
    return nf4_lora_wgrad_multi_workspace(&j, 1, m, rank);
}

extern "C" int nf4_lora_wgrad(const void *u, int64_t m, int64_t p, int64_t ldu, const void *v,
                              int rank, float scale, float *out, int transpose_out, int dtype,
                              void *workspace, size_t workspace_bytes, void *stream) {
    if (!out || (m > 0 && p > 0 && (!u || !v))) return NF4_ERR_ARG;
    const nf4_lora_job j = {u, ldu, p, v, out, scale, transpose_out};
    return nf4_lora_wgrad_multi(&j, 1, m, rank, dtype, workspace, workspace_bytes, stream);
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
        hipLaunchKernelGGL(swiglu_fwd_kernel<NF4_BF16>, grid_2d(rows, cols), dim3(256), 0, s, g, u,
                           ld_gu, o, ld_h, rows, cols);
    else
        hipLaunchKernelGGL(swiglu_fwd_kernel<NF4_F16>, grid_2d(rows, cols), dim3(256), 0, s, g, u,
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
        hipLaunchKernelGGL(swiglu_bwd_kernel<NF4_BF16>, grid_2d(rows, cols), dim3(256), 0, s, d,
                           ld_h, g, u, ld_gu, dg, du, rows, cols);
    else
        hipLaunchKernelGGL(swiglu_bwd_kernel<NF4_F16>, grid_2d(rows, cols), dim3(256), 0, s, d,
                           ld_h, g, u, ld_gu, dg, du, rows, cols);
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
    // Workspace-free and deterministic: a workgroup per 64 columns, rows split over its threads
    // in a fixed way and the row-lane sums added in order.
    const int vec = n % 8 == 0 && lddy % 8 == 0 && aligned(dy, 16);
    const dim3 grid(static_cast<unsigned>((n + kColsumCols - 1) / kColsumCols));
    const auto d = static_cast<const uint16_t *>(dy);
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL(colsum_kernel<NF4_BF16>, grid, dim3(256), 0, s, d, m, n, lddy, vec, out);
    else
        hipLaunchKernelGGL(colsum_kernel<NF4_F16>, grid, dim3(256), 0, s, d, m, n, lddy, vec, out);
    return status_of(hipGetLastError());
}
