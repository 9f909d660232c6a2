// The neighbours of the q|k|v projection in a decoder layer, for gfx950: the RMSNorm that
// produces the projection's input (and LoRA's dropout-masked inputs) and the rotary embedding
// that consumes its output, forward and backward.
//
// Reference: add_rmsnorm_fwd_kernel, rmsnorm_bwd_lora_kernel, qkv_lora_rope_kernel and
// qkv_rope_bwd_kernel (/root/reference/solution/layer.py:92-132, 135-164, 167-218, 221-263).
// The interface differs in one place: the reference adds the LoRA outputs of q and v inside its
// RoPE kernel (layer.py:190-193, 208-211); here the projection GEMM adds them in its epilogue
// (nf4_linear_fwd with LoRA slabs), so the RoPE kernel reads the finished q|k|v.
// Every kernel computes in fp32 and rounds once per output; all are bound by HBM traffic.

#include <initializer_list>

#include "nf4_common.h"

namespace {

template <int DT>
__device__ __forceinline__ float bits_f32(uint16_t b) {
    if constexpr (DT == NF4_BF16) return __uint_as_float(static_cast<uint32_t>(b) << 16);
    else return static_cast<float>(__builtin_bit_cast(half_t, b));
}

template <int DT>
__device__ __forceinline__ float ld1(const uint16_t *p) {
    return bits_f32<DT>(*p);
}

template <int DT>
__device__ __forceinline__ uint16_t st1(float v) {
    return round16<DT>(v);
}

// 8 consecutive 16-bit values <-> 8 floats (one 16-byte access).
template <int DT>
__device__ __forceinline__ void load8(const uint16_t *p, float (&v)[8]) {
    const u32x4_t r = *reinterpret_cast<const u32x4_t *>(p);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = bits_f32<DT>(static_cast<uint16_t>(w[i] & 0xffffu));
        v[2 * i + 1] = bits_f32<DT>(static_cast<uint16_t>(w[i] >> 16));
    }
}

template <int DT>
__device__ __forceinline__ void store8(uint16_t *p, const float (&v)[8]) {
    u32x4_t r;
    r.x = st1<DT>(v[0]) | (static_cast<uint32_t>(st1<DT>(v[1])) << 16);
    r.y = st1<DT>(v[2]) | (static_cast<uint32_t>(st1<DT>(v[3])) << 16);
    r.z = st1<DT>(v[4]) | (static_cast<uint32_t>(st1<DT>(v[5])) << 16);
    r.w = st1<DT>(v[6]) | (static_cast<uint32_t>(st1<DT>(v[7])) << 16);
    *reinterpret_cast<u32x4_t *>(p) = r;
}

constexpr int kNormThreads = 256;
constexpr int kNormChunks = 4;  // 8-element chunks per thread: rows up to 8192 elements

// 8 consecutive values of the residual stream (fp32, or the GEMM dtype when RT == DT) <-> 8
// floats.
template <int DT, int RT>
__device__ __forceinline__ void load8r(const void *p, int64_t o, float (&v)[8]) {
    if constexpr (RT == NF4_F32) {
        const float4_t a = *reinterpret_cast<const float4_t *>(static_cast<const float *>(p) + o);
        const float4_t b = *reinterpret_cast<const float4_t *>(static_cast<const float *>(p) + o + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = a[i];
            v[4 + i] = b[i];
        }
    } else {
        load8<DT>(static_cast<const uint16_t *>(p) + o, v);
    }
}

template <int DT, int RT>
__device__ __forceinline__ void store8r(void *p, int64_t o, const float (&v)[8]) {
    if constexpr (RT == NF4_F32) {
        float *q = static_cast<float *>(p) + o;
        *reinterpret_cast<float4_t *>(q) = (float4_t){v[0], v[1], v[2], v[3]};
        *reinterpret_cast<float4_t *>(q + 4) = (float4_t){v[4], v[5], v[6], v[7]};
    } else {
        store8<DT>(static_cast<uint16_t *>(p) + o, v);
    }
}

// The packed keep bits of one 8-element chunk: bit i of the byte = element i (layer.py:76-90).
__device__ __forceinline__ uint32_t pack8(const uint8_t *keep) {
    const u32x2_t k = *reinterpret_cast<const u32x2_t *>(keep);
    uint32_t b = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        b |= ((k.x >> (8 * i)) & 1u) << i;
        b |= ((k.y >> (8 * i)) & 1u) << (4 + i);
    }
    return b;
}

// Sum over the workgroup (4 waves): wave reductions through cross-lane shuffles, then the four
// wave sums in LDS in wave order, so every thread gets the same value.
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

struct NormDrop {
    const uint8_t *keep_q, *keep_v;  // mode 1: one byte per element, rows src_rows[r] (or r)
    const int64_t *src_rows;
    int64_t keep_rows;               // mode 1: rows of keep_q / keep_v
    uint8_t *packed;                 // [rows][2][cols / 8]: q's bits, then v's
    int mode;                        // 0 none, 1 pack from keep_q / keep_v, 2 read packed
    float scale_q, scale_v;
};

// One row per workgroup (layer.py:92-132): h = x (+ d) in fp32, rstd = 1 / sqrt(mean(h^2)
// + eps), y = w * (h * rstd) rounded to DT; with dropout also LoRA's two inputs
// oq = y * keep_q * scale_q and ov = y * keep_v * scale_v, each rounded once.  A thread's
// 8-element chunk ch is bit byte ch of the row's packed masks.  x is the residual stream in RT
// (fp32 or DT), d the output of o_proj in DT.
template <int DT, int RT>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(
    const void *x, const uint16_t *d, const float *w, uint16_t *y, float *rstd_out,
    const NormDrop drop, uint16_t *oq, uint16_t *ov, int64_t cols, float eps) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const int64_t base = row * cols;
    const int chunks = static_cast<int>(cols / 8);
    float h[kNormChunks][8];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
        const int ch = threadIdx.x + c * kNormThreads;
        if (ch >= chunks) continue;
        load8r<DT, RT>(x, base + ch * 8, h[c]);
        if (d) {
            float e[8];
            load8<DT>(d + base + ch * 8, e);
#pragma unroll
            for (int i = 0; i < 8; ++i) h[c][i] += e[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += h[c][i] * h[c][i];
    }
    ss = block_sum(ss, red);
    const float rstd = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
    if (threadIdx.x == 0) rstd_out[row] = rstd;
    const int64_t src = drop.mode == 1 && drop.src_rows ? drop.src_rows[row] : row;
    // a mask row outside keep_q / keep_v (a bad row map) is read as all dropped, never fetched
    const bool src_ok = src >= 0 && src < drop.keep_rows;
    uint8_t *bits = drop.mode != 0 ? drop.packed + row * 2 * chunks : nullptr;
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
        const int ch = threadIdx.x + c * kNormThreads;
        if (ch >= chunks) continue;
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = w[ch * 8 + i] * (h[c][i] * rstd);
        store8<DT>(y + base + ch * 8, v);
        if (drop.mode != 0) {
            uint32_t bq, bv;
            if (drop.mode == 1) {
                bq = src_ok ? pack8(drop.keep_q + src * cols + ch * 8) : 0u;
                bv = src_ok ? pack8(drop.keep_v + src * cols + ch * 8) : 0u;
                bits[ch] = static_cast<uint8_t>(bq);
                bits[chunks + ch] = static_cast<uint8_t>(bv);
            } else {
                bq = bits[ch];
                bv = bits[chunks + ch];
            }
            float q[8], vv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                q[i] = v[i] * static_cast<float>((bq >> i) & 1u) * drop.scale_q;
                vv[i] = v[i] * static_cast<float>((bv >> i) & 1u) * drop.scale_v;
            }
            store8<DT>(oq + base + ch * 8, q);
            store8<DT>(ov + base + ch * 8, vv);
        }
    }
}

// One row per workgroup (layer.py:135-164): g = dy (+ dq * keep_q * scale_q
// + dv * keep_v * scale_v, keep bits from the packed masks), h = x (+ d) recomputed,
// h^ = h * rstd, gw = g * w, dx = rstd * (gw - h^ * mean(gw * h^)) (+ dres).  x, dres and dx
// are the residual stream in RT; dy, dq, dv and d in DT.
template <int DT, int RT>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_bwd_kernel(
    const uint16_t *dy, const uint16_t *dq, const uint16_t *dv, const uint8_t *packed,
    float scale_q, float scale_v, const void *x, const uint16_t *d, const float *w,
    const float *rstd_in, const void *dres, void *dx, int64_t cols) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const int64_t base = row * cols;
    const int chunks = static_cast<int>(cols / 8);
    const float rstd = rstd_in[row];
    const uint8_t *bits = dq ? packed + row * 2 * chunks : nullptr;
    float gw[kNormChunks][8], hh[kNormChunks][8];
    float proj = 0.f;
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
        const int ch = threadIdx.x + c * kNormThreads;
        if (ch >= chunks) continue;
        const int64_t o = base + ch * 8;
        float g[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (dy) load8<DT>(dy + o, g);
        if (dq) {
            float a[8], b[8];
            load8<DT>(dq + o, a);
            load8<DT>(dv + o, b);
            const uint32_t bq = bits[ch], bv = bits[chunks + ch];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                g[i] += a[i] * static_cast<float>((bq >> i) & 1u) * scale_q;
                g[i] += b[i] * static_cast<float>((bv >> i) & 1u) * scale_v;
            }
        }
        load8r<DT, RT>(x, o, hh[c]);
        if (d) {
            float e[8];
            load8<DT>(d + o, e);
#pragma unroll
            for (int i = 0; i < 8; ++i) hh[c][i] += e[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            hh[c][i] *= rstd;
            gw[c][i] = g[i] * w[ch * 8 + i];
            proj += gw[c][i] * hh[c][i];
        }
    }
    proj = block_sum(proj, red) / static_cast<float>(cols);
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
        const int ch = threadIdx.x + c * kNormThreads;
        if (ch >= chunks) continue;
        const int64_t o = base + ch * 8;
        float v[8], r[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (dres) load8r<DT, RT>(dres, o, r);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = rstd * (gw[c][i] - hh[c][i] * proj) + r[i];
        store8r<DT, RT>(dx, o, v);
    }
}

// Program (token, query head), one lane per rotary pair i < head_dim / 2 (layer.py:167-218):
// q and k rotated in fp32 (lo' = lo cos_lo - hi sin_lo, hi' = hi cos_hi + lo sin_hi), k and v
// expanded to every query head of their group ([tokens, heads, dim]), and the unexpanded k, v
// written once per group when caches are given.
template <int DT>
__global__ __launch_bounds__(64) void qkv_rope_kernel(
    const uint16_t *qkv, int64_t ld, const float *cs, const float *sn, uint16_t *qe, uint16_t *ke,
    uint16_t *ve, uint16_t *kc, uint16_t *vc, int n_heads, int n_kv, int head_dim) {
    const int64_t t = blockIdx.x;
    const int head = blockIdx.y, groups = n_heads / n_kv, kv = head / groups, half = head_dim / 2;
    const uint16_t *src = qkv + t * ld;
    const int64_t dst = (t * n_heads + head) * head_dim;
    const int64_t cdst = (t * n_kv + kv) * head_dim;
    for (int i = threadIdx.x; i < half; i += 64) {
        const float c_lo = cs[t * head_dim + i], c_hi = cs[t * head_dim + half + i];
        const float s_lo = sn[t * head_dim + i], s_hi = sn[t * head_dim + half + i];
        float lo = ld1<DT>(src + head * head_dim + i), hi = ld1<DT>(src + head * head_dim + half + i);
        qe[dst + i] = st1<DT>(lo * c_lo - hi * s_lo);
        qe[dst + half + i] = st1<DT>(hi * c_hi + lo * s_hi);
        const int ko = (n_heads + kv) * head_dim;
        lo = ld1<DT>(src + ko + i);
        hi = ld1<DT>(src + ko + half + i);
        const uint16_t k_lo = st1<DT>(lo * c_lo - hi * s_lo), k_hi = st1<DT>(hi * c_hi + lo * s_hi);
        ke[dst + i] = k_lo;
        ke[dst + half + i] = k_hi;
        const int vo = (n_heads + n_kv + kv) * head_dim;
        const uint16_t v_lo = src[vo + i], v_hi = src[vo + half + i];
        ve[dst + i] = v_lo;
        ve[dst + half + i] = v_hi;
        if (head % groups == 0 && kc) {
            kc[cdst + i] = k_lo;
            kc[cdst + half + i] = k_hi;
            vc[cdst + i] = v_lo;
            vc[cdst + half + i] = v_hi;
        }
    }
}

// Program (token, query head or key/value head) (layer.py:221-263): the transposed rotation of
// the gradients into the [tokens, q|k|v] layout; a key/value head first sums the gradients of
// its expanded copies in head order.
template <int DT>
__global__ __launch_bounds__(64) void qkv_rope_bwd_kernel(
    const uint16_t *dqe, const uint16_t *dke, const uint16_t *dve, const float *cs, const float *sn,
    uint16_t *dqkv, int64_t ld, int n_heads, int n_kv, int head_dim) {
    const int64_t t = blockIdx.x;
    const int head = blockIdx.y, groups = n_heads / n_kv, half = head_dim / 2;
    uint16_t *dst = dqkv + t * ld;
    for (int i = threadIdx.x; i < half; i += 64) {
        const float c_lo = cs[t * head_dim + i], c_hi = cs[t * head_dim + half + i];
        const float s_lo = sn[t * head_dim + i], s_hi = sn[t * head_dim + half + i];
        if (head < n_heads) {
            const int64_t s = (t * n_heads + head) * head_dim;
            const float g_lo = ld1<DT>(dqe + s + i), g_hi = ld1<DT>(dqe + s + half + i);
            dst[head * head_dim + i] = st1<DT>(g_lo * c_lo + g_hi * s_hi);
            dst[head * head_dim + half + i] = st1<DT>(g_hi * c_hi - g_lo * s_lo);
        } else {
            const int kv = head - n_heads;
            float k_lo = 0.f, k_hi = 0.f, v_lo = 0.f, v_hi = 0.f;
            for (int r = 0; r < groups; ++r) {
                const int64_t s = (t * n_heads + kv * groups + r) * head_dim;
                k_lo += ld1<DT>(dke + s + i);
                k_hi += ld1<DT>(dke + s + half + i);
                v_lo += ld1<DT>(dve + s + i);
                v_hi += ld1<DT>(dve + s + half + i);
            }
            const int ko = (n_heads + kv) * head_dim, vo = (n_heads + n_kv + kv) * head_dim;
            dst[ko + i] = st1<DT>(k_lo * c_lo + k_hi * s_hi);
            dst[ko + half + i] = st1<DT>(k_hi * c_hi - k_lo * s_lo);
            dst[vo + i] = st1<DT>(v_lo);
            dst[vo + half + i] = st1<DT>(v_hi);
        }
    }
}

// Vector forms for head_dim a multiple of 8 (up to 512): a lane takes 4 consecutive rotary
// pairs (8-byte accesses of lo and hi, 16-byte cos / sin), so one wave covers 256 / head_dim
// heads, or one head in head_dim / 256 passes.  Same arithmetic as the scalar kernels.
template <int DT>
__device__ __forceinline__ void ld4(const uint16_t *p, float (&v)[4]) {
    const u32x2_t r = *reinterpret_cast<const u32x2_t *>(p);
    v[0] = bits_f32<DT>(static_cast<uint16_t>(r.x & 0xffffu));
    v[1] = bits_f32<DT>(static_cast<uint16_t>(r.x >> 16));
    v[2] = bits_f32<DT>(static_cast<uint16_t>(r.y & 0xffffu));
    v[3] = bits_f32<DT>(static_cast<uint16_t>(r.y >> 16));
}

__device__ __forceinline__ u32x2_t pack4(const uint16_t (&v)[4]) {
    return (u32x2_t){v[0] | (static_cast<uint32_t>(v[1]) << 16),
                     v[2] | (static_cast<uint32_t>(v[3]) << 16)};
}

__device__ __forceinline__ void ldf4(const float *p, float (&v)[4]) {
    const float4_t r = *reinterpret_cast<const float4_t *>(p);
    v[0] = r.x;
    v[1] = r.y;
    v[2] = r.z;
    v[3] = r.w;
}

// Grid: x = tokens, y = groups of heads per wave.  Lane l: head (y * hpw + l / lph), pairs
// 4 (l % lph) .. + 3 (lph = lanes per head).
template <int DT>
__global__ __launch_bounds__(64) void qkv_rope_vec_kernel(
    const uint16_t *qkv, int64_t ld, const float *cs, const float *sn, uint16_t *qe, uint16_t *ke,
    uint16_t *ve, uint16_t *kc, uint16_t *vc, int n_heads, int n_kv, int head_dim) {
    const int64_t t = blockIdx.x;
    const int half = head_dim / 2, lph = half / 4 < 64 ? half / 4 : 64, hpw = 64 / lph;
    const int head = blockIdx.y * hpw + threadIdx.x / lph;
    if (head >= n_heads) return;
    const int groups = n_heads / n_kv, kv = head / groups;
    const uint16_t *src = qkv + t * ld;
    const int64_t dst = (t * n_heads + head) * head_dim;
    const int64_t cdst = (t * n_kv + kv) * head_dim;
    for (int i = (threadIdx.x % lph) * 4; i < half; i += lph * 4) {
        float c_lo[4], c_hi[4], s_lo[4], s_hi[4], lo[4], hi[4];
        ldf4(cs + t * head_dim + i, c_lo);
        ldf4(cs + t * head_dim + half + i, c_hi);
        ldf4(sn + t * head_dim + i, s_lo);
        ldf4(sn + t * head_dim + half + i, s_hi);
        uint16_t a[4], b[4];
        ld4<DT>(src + head * head_dim + i, lo);
        ld4<DT>(src + head * head_dim + half + i, hi);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a[j] = st1<DT>(lo[j] * c_lo[j] - hi[j] * s_lo[j]);
            b[j] = st1<DT>(hi[j] * c_hi[j] + lo[j] * s_hi[j]);
        }
        *reinterpret_cast<u32x2_t *>(qe + dst + i) = pack4(a);
        *reinterpret_cast<u32x2_t *>(qe + dst + half + i) = pack4(b);
        const int ko = (n_heads + kv) * head_dim, vo = (n_heads + n_kv + kv) * head_dim;
        ld4<DT>(src + ko + i, lo);
        ld4<DT>(src + ko + half + i, hi);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a[j] = st1<DT>(lo[j] * c_lo[j] - hi[j] * s_lo[j]);
            b[j] = st1<DT>(hi[j] * c_hi[j] + lo[j] * s_hi[j]);
        }
        const u32x2_t klo = pack4(a), khi = pack4(b);
        const u32x2_t vlo = *reinterpret_cast<const u32x2_t *>(src + vo + i);
        const u32x2_t vhi = *reinterpret_cast<const u32x2_t *>(src + vo + half + i);
        *reinterpret_cast<u32x2_t *>(ke + dst + i) = klo;
        *reinterpret_cast<u32x2_t *>(ke + dst + half + i) = khi;
        *reinterpret_cast<u32x2_t *>(ve + dst + i) = vlo;
        *reinterpret_cast<u32x2_t *>(ve + dst + half + i) = vhi;
        if (head % groups == 0 && kc) {
            *reinterpret_cast<u32x2_t *>(kc + cdst + i) = klo;
            *reinterpret_cast<u32x2_t *>(kc + cdst + half + i) = khi;
            *reinterpret_cast<u32x2_t *>(vc + cdst + i) = vlo;
            *reinterpret_cast<u32x2_t *>(vc + cdst + half + i) = vhi;
        }
    }
}

// Grid: x = tokens, y = groups of (query or key/value) heads per wave, heads numbered as in
// qkv_rope_bwd_kernel.
constexpr int kRopeGroupBatch = 8;

template <int DT>
__global__ __launch_bounds__(64) void qkv_rope_bwd_vec_kernel(
    const uint16_t *dqe, const uint16_t *dke, const uint16_t *dve, const float *cs, const float *sn,
    uint16_t *dqkv, int64_t ld, int n_heads, int n_kv, int head_dim) {
    const int64_t t = blockIdx.x;
    const int half = head_dim / 2, lph = half / 4 < 64 ? half / 4 : 64, hpw = 64 / lph;
    const int head = blockIdx.y * hpw + threadIdx.x / lph;
    if (head >= n_heads + n_kv) return;
    const int groups = n_heads / n_kv;
    uint16_t *dst = dqkv + t * ld;
    for (int i = (threadIdx.x % lph) * 4; i < half; i += lph * 4) {
        float c_lo[4], c_hi[4], s_lo[4], s_hi[4];
        ldf4(cs + t * head_dim + i, c_lo);
        ldf4(cs + t * head_dim + half + i, c_hi);
        ldf4(sn + t * head_dim + i, s_lo);
        ldf4(sn + t * head_dim + half + i, s_hi);
        uint16_t a[4], b[4];
        if (head < n_heads) {
            const int64_t s = (t * n_heads + head) * head_dim;
            float g_lo[4], g_hi[4];
            ld4<DT>(dqe + s + i, g_lo);
            ld4<DT>(dqe + s + half + i, g_hi);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                a[j] = st1<DT>(g_lo[j] * c_lo[j] + g_hi[j] * s_hi[j]);
                b[j] = st1<DT>(g_hi[j] * c_hi[j] - g_lo[j] * s_lo[j]);
            }
            *reinterpret_cast<u32x2_t *>(dst + head * head_dim + i) = pack4(a);
            *reinterpret_cast<u32x2_t *>(dst + head * head_dim + half + i) = pack4(b);
        } else {
            const int kv = head - n_heads;
            float k_lo[4] = {0.f, 0.f, 0.f, 0.f}, k_hi[4] = {0.f, 0.f, 0.f, 0.f};
            float v_lo[4] = {0.f, 0.f, 0.f, 0.f}, v_hi[4] = {0.f, 0.f, 0.f, 0.f};
            // the query heads of this kv head in batches of kRopeGroupBatch: every load of a
            // batch is issued before its sums (in head order), so the lane waits for one memory
            // latency per batch instead of one per head
            for (int r0 = 0; r0 < groups; r0 += kRopeGroupBatch) {
                u32x2_t e[kRopeGroupBatch][4];
#pragma unroll
                for (int r = 0; r < kRopeGroupBatch; ++r) {
                    if (r0 + r >= groups) break;
                    const int64_t s = (t * n_heads + kv * groups + r0 + r) * head_dim;
                    e[r][0] = *reinterpret_cast<const u32x2_t *>(dke + s + i);
                    e[r][1] = *reinterpret_cast<const u32x2_t *>(dke + s + half + i);
                    e[r][2] = *reinterpret_cast<const u32x2_t *>(dve + s + i);
                    e[r][3] = *reinterpret_cast<const u32x2_t *>(dve + s + half + i);
                }
#pragma unroll
                for (int r = 0; r < kRopeGroupBatch; ++r) {
                    if (r0 + r >= groups) break;
                    float f[4][4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        f[u][0] = bits_f32<DT>(static_cast<uint16_t>(e[r][u].x & 0xffffu));
                        f[u][1] = bits_f32<DT>(static_cast<uint16_t>(e[r][u].x >> 16));
                        f[u][2] = bits_f32<DT>(static_cast<uint16_t>(e[r][u].y & 0xffffu));
                        f[u][3] = bits_f32<DT>(static_cast<uint16_t>(e[r][u].y >> 16));
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        k_lo[j] += f[0][j];
                        k_hi[j] += f[1][j];
                        v_lo[j] += f[2][j];
                        v_hi[j] += f[3][j];
                    }
                }
            }
            const int ko = (n_heads + kv) * head_dim, vo = (n_heads + n_kv + kv) * head_dim;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                a[j] = st1<DT>(k_lo[j] * c_lo[j] + k_hi[j] * s_hi[j]);
                b[j] = st1<DT>(k_hi[j] * c_hi[j] - k_lo[j] * s_lo[j]);
            }
            *reinterpret_cast<u32x2_t *>(dst + ko + i) = pack4(a);
            *reinterpret_cast<u32x2_t *>(dst + ko + half + i) = pack4(b);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                a[j] = st1<DT>(v_lo[j]);
                b[j] = st1<DT>(v_hi[j]);
            }
            *reinterpret_cast<u32x2_t *>(dst + vo + i) = pack4(a);
            *reinterpret_cast<u32x2_t *>(dst + vo + half + i) = pack4(b);
        }
    }
}

int norm_shape_ok(int64_t rows, int64_t cols, int dtype) {
    if (dtype != NF4_F16 && dtype != NF4_BF16) return NF4_ERR_ARG;
    if (rows < 0 || cols <= 0) return NF4_ERR_ARG;
    if (cols % 8 != 0 || cols > 8LL * kNormThreads * kNormChunks) return NF4_ERR_UNSUPPORTED;
    return NF4_OK;
}

// The vector kernels: head_dim a multiple of 8 up to 512, 8-byte aligned 16-bit tensors with a
// row stride of a multiple of 4 elements, 16-byte aligned cos / sin.
bool rope_vec_ok(int head_dim, int64_t ld, std::initializer_list<const void *> ptrs,
                 const float *c, const float *s) {
    if (head_dim % 8 != 0 || head_dim > 512 || ld % 4 != 0) return false;
    for (const void *p : ptrs)
        if (p && !aligned(p, 8)) return false;
    return aligned(c, 16) && aligned(s, 16);
}

int rope_shape_ok(int64_t tokens, int n_heads, int n_kv, int head_dim, int dtype) {
    if (dtype != NF4_F16 && dtype != NF4_BF16) return NF4_ERR_ARG;
    if (tokens < 0 || n_heads < 1 || n_kv < 1 || head_dim < 2 || head_dim % 2) return NF4_ERR_ARG;
    if (n_heads % n_kv != 0 || tokens > 0x7fffffff || n_heads + n_kv > 65535) return NF4_ERR_ARG;
    return NF4_OK;
}

}  // namespace

extern "C" int nf4_add_rmsnorm(const void *x, int res_dtype, const void *d, const float *w,
                               void *y, float *rstd, const uint8_t *keep_q,
                               const uint8_t *keep_v, const int64_t *src_rows, int64_t keep_rows,
                               uint8_t *packed, int drop_mode, float scale_q, float scale_v,
                               void *oq, void *ov, int64_t rows, int64_t cols, float eps,
                               int dtype, void *stream) {
    int st = norm_shape_ok(rows, cols, dtype);
    if (st != NF4_OK) return st;
    if (res_dtype != dtype && res_dtype != NF4_F32) return NF4_ERR_ARG;
    if (rows > 0 && (!x || !w || !y || !rstd)) return NF4_ERR_ARG;
    if (drop_mode < 0 || drop_mode > 2) return NF4_ERR_ARG;
    if (drop_mode != 0 && (!packed || !oq || !ov)) return NF4_ERR_ARG;
    if (drop_mode == 1 && (!keep_q || !keep_v || keep_rows < 0)) return NF4_ERR_ARG;
    if (drop_mode == 1 && !src_rows && keep_rows < rows) return NF4_ERR_ARG;  // masks row r
    for (const void *p : {x, d, static_cast<const void *>(y), static_cast<const void *>(oq),
                          static_cast<const void *>(ov)})
        if (p && !aligned(p, 16)) return NF4_ERR_UNSUPPORTED;
    if (drop_mode == 1 && (!aligned(keep_q, 8) || !aligned(keep_v, 8))) return NF4_ERR_UNSUPPORTED;
    if (rows == 0) return NF4_OK;
    if (rows > 0x7fffffff) return NF4_ERR_ARG;
    auto s = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(rows));
    const NormDrop dr{keep_q, keep_v, src_rows, keep_rows, packed, drop_mode, scale_q, scale_v};
    auto D = static_cast<const uint16_t *>(d);
    auto Y = static_cast<uint16_t *>(y), Q = static_cast<uint16_t *>(oq), V = static_cast<uint16_t *>(ov);
#define NF4_NORM_FWD(DT, RT)                                                                       \
    hipLaunchKernelGGL((add_rmsnorm_kernel<DT, RT>), grid, dim3(kNormThreads), 0, s, x, D, w, Y,  \
                       rstd, dr, Q, V, cols, eps)
    if (dtype == NF4_BF16) {
        if (res_dtype == NF4_F32) NF4_NORM_FWD(NF4_BF16, NF4_F32);
        else NF4_NORM_FWD(NF4_BF16, NF4_BF16);
    } else {
        if (res_dtype == NF4_F32) NF4_NORM_FWD(NF4_F16, NF4_F32);
        else NF4_NORM_FWD(NF4_F16, NF4_F16);
    }
#undef NF4_NORM_FWD
    return status_of(hipGetLastError());
}

extern "C" int nf4_rmsnorm_bwd(const void *dy, const void *dq, const void *dv,
                               const uint8_t *packed, float scale_q, float scale_v, const void *x,
                               int res_dtype, const void *d, const float *w, const float *rstd,
                               const void *dres, void *dx, int64_t rows, int64_t cols, int dtype,
                               void *stream) {
    int st = norm_shape_ok(rows, cols, dtype);
    if (st != NF4_OK) return st;
    if (res_dtype != dtype && res_dtype != NF4_F32) return NF4_ERR_ARG;
    if (rows > 0 && (!x || !w || !rstd || !dx)) return NF4_ERR_ARG;
    if ((dq != nullptr) != (dv != nullptr) || (dq && !packed)) return NF4_ERR_ARG;
    for (const void *p : {dy, dq, dv, x, d, dres, static_cast<const void *>(dx)})
        if (p && !aligned(p, 16)) return NF4_ERR_UNSUPPORTED;
    if (rows == 0) return NF4_OK;
    if (rows > 0x7fffffff) return NF4_ERR_ARG;
    auto s = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(rows));
    auto P = [](const void *p) { return static_cast<const uint16_t *>(p); };
#define NF4_NORM_BWD(DT, RT)                                                                       \
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<DT, RT>), grid, dim3(kNormThreads), 0, s, P(dy), P(dq), \
                       P(dv), packed, scale_q, scale_v, x, P(d), w, rstd, dres, dx, cols)
    if (dtype == NF4_BF16) {
        if (res_dtype == NF4_F32) NF4_NORM_BWD(NF4_BF16, NF4_F32);
        else NF4_NORM_BWD(NF4_BF16, NF4_BF16);
    } else {
        if (res_dtype == NF4_F32) NF4_NORM_BWD(NF4_F16, NF4_F32);
        else NF4_NORM_BWD(NF4_F16, NF4_F16);
    }
#undef NF4_NORM_BWD
    return status_of(hipGetLastError());
}

extern "C" int nf4_qkv_rope(const void *qkv, int64_t ld_qkv, const float *cos_t, const float *sin_t,
                            void *q, void *k, void *v, void *k_cache, void *v_cache,
                            int64_t tokens, int n_heads, int n_kv, int head_dim, int dtype,
                            void *stream) {
    int st = rope_shape_ok(tokens, n_heads, n_kv, head_dim, dtype);
    if (st != NF4_OK) return st;
    if (tokens > 0 && (!qkv || !cos_t || !sin_t || !q || !k || !v)) return NF4_ERR_ARG;
    if ((k_cache != nullptr) != (v_cache != nullptr)) return NF4_ERR_ARG;
    if (ld_qkv < static_cast<int64_t>(n_heads + 2 * n_kv) * head_dim) return NF4_ERR_ARG;
    if (tokens == 0) return NF4_OK;
    auto s = static_cast<hipStream_t>(stream);
    auto P = [](void *p) { return static_cast<uint16_t *>(p); };
    if (rope_vec_ok(head_dim, ld_qkv, {qkv, q, k, v, k_cache, v_cache}, cos_t, sin_t)) {
        const int lph = head_dim / 8 < 64 ? head_dim / 8 : 64, hpw = 64 / lph;
        const dim3 vgrid(static_cast<unsigned>(tokens), static_cast<unsigned>((n_heads + hpw - 1) / hpw));
        if (dtype == NF4_BF16)
            hipLaunchKernelGGL(qkv_rope_vec_kernel<NF4_BF16>, vgrid, dim3(64), 0, s,
                               static_cast<const uint16_t *>(qkv), ld_qkv, cos_t, sin_t, P(q), P(k),
                               P(v), P(k_cache), P(v_cache), n_heads, n_kv, head_dim);
        else
            hipLaunchKernelGGL(qkv_rope_vec_kernel<NF4_F16>, vgrid, dim3(64), 0, s,
                               static_cast<const uint16_t *>(qkv), ld_qkv, cos_t, sin_t, P(q), P(k),
                               P(v), P(k_cache), P(v_cache), n_heads, n_kv, head_dim);
        return status_of(hipGetLastError());
    }
    const dim3 grid(static_cast<unsigned>(tokens), static_cast<unsigned>(n_heads));
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL(qkv_rope_kernel<NF4_BF16>, grid, dim3(64), 0, s,
                           static_cast<const uint16_t *>(qkv), ld_qkv, cos_t, sin_t, P(q), P(k),
                           P(v), P(k_cache), P(v_cache), n_heads, n_kv, head_dim);
    else
        hipLaunchKernelGGL(qkv_rope_kernel<NF4_F16>, grid, dim3(64), 0, s,
                           static_cast<const uint16_t *>(qkv), ld_qkv, cos_t, sin_t, P(q), P(k),
                           P(v), P(k_cache), P(v_cache), n_heads, n_kv, head_dim);
    return status_of(hipGetLastError());
}

extern "C" int nf4_qkv_rope_bwd(const void *dq, const void *dk, const void *dv, const float *cos_t,
                                const float *sin_t, void *dqkv, int64_t ld_dqkv, int64_t tokens,
                                int n_heads, int n_kv, int head_dim, int dtype, void *stream) {
    int st = rope_shape_ok(tokens, n_heads, n_kv, head_dim, dtype);
    if (st != NF4_OK) return st;
    if (tokens > 0 && (!dq || !dk || !dv || !cos_t || !sin_t || !dqkv)) return NF4_ERR_ARG;
    if (ld_dqkv < static_cast<int64_t>(n_heads + 2 * n_kv) * head_dim) return NF4_ERR_ARG;
    if (tokens == 0) return NF4_OK;
    auto s = static_cast<hipStream_t>(stream);
    auto P = [](const void *p) { return static_cast<const uint16_t *>(p); };
    if (rope_vec_ok(head_dim, ld_dqkv, {dq, dk, dv, dqkv}, cos_t, sin_t)) {
        const int lph = head_dim / 8 < 64 ? head_dim / 8 : 64, hpw = 64 / lph;
        const dim3 vgrid(static_cast<unsigned>(tokens),
                         static_cast<unsigned>((n_heads + n_kv + hpw - 1) / hpw));
        if (dtype == NF4_BF16)
            hipLaunchKernelGGL(qkv_rope_bwd_vec_kernel<NF4_BF16>, vgrid, dim3(64), 0, s, P(dq), P(dk),
                               P(dv), cos_t, sin_t, static_cast<uint16_t *>(dqkv), ld_dqkv, n_heads,
                               n_kv, head_dim);
        else
            hipLaunchKernelGGL(qkv_rope_bwd_vec_kernel<NF4_F16>, vgrid, dim3(64), 0, s, P(dq), P(dk),
                               P(dv), cos_t, sin_t, static_cast<uint16_t *>(dqkv), ld_dqkv, n_heads,
                               n_kv, head_dim);
        return status_of(hipGetLastError());
    }
    const dim3 grid(static_cast<unsigned>(tokens), static_cast<unsigned>(n_heads + n_kv));
    if (dtype == NF4_BF16)
        hipLaunchKernelGGL(qkv_rope_bwd_kernel<NF4_BF16>, grid, dim3(64), 0, s, P(dq), P(dk), P(dv),
                           cos_t, sin_t, static_cast<uint16_t *>(dqkv), ld_dqkv, n_heads, n_kv,
                           head_dim);
    else
        hipLaunchKernelGGL(qkv_rope_bwd_kernel<NF4_F16>, grid, dim3(64), 0, s, P(dq), P(dk), P(dv),
                           cos_t, sin_t, static_cast<uint16_t *>(dqkv), ld_dqkv, n_heads, n_kv,
                           head_dim);
    return status_of(hipGetLastError());
}
