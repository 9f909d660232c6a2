// Shared device-side definitions of the gfx950 NF4 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nf4_mi355x.h"

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16_t;
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf168_t __attribute__((ext_vector_type(8)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Device copy of nf4_weight with the element count precomputed.
struct DevWeight {
    const uint8_t *packed;
    const void *absmax;
    const float *absmax2;
    const float *code2;
    const float *code;
    float offset;
    int32_t nested;
    int64_t rows;
    int64_t cols;
    int32_t blocksize;
    int32_t blocksize2;
    int32_t bs_shift;   // log2(blocksize) if a power of two, else -1
    int32_t bs2_shift;  // log2(blocksize2) if a power of two, else -1
};

static inline int log2_exact(int64_t v) {
    if (v <= 0 || (v & (v - 1))) return -1;
    int s = 0;
    while ((int64_t(1) << s) < v) ++s;
    return s;
}

static inline DevWeight to_dev(const nf4_weight &w) {
    DevWeight d;
    d.packed = w.packed;
    d.absmax = w.absmax;
    d.absmax2 = w.absmax2;
    d.code2 = w.code2;
    d.code = w.code;
    d.offset = w.offset;
    d.nested = w.nested;
    d.rows = w.rows;
    d.cols = w.cols;
    d.blocksize = w.blocksize;
    d.blocksize2 = w.blocksize2;
    d.bs_shift = log2_exact(w.blocksize);
    d.bs2_shift = log2_exact(w.blocksize2);
    return d;
}

// Absmax block of element e and absmax2 group of block b: shifts for power-of-two sizes (every
// blocksize bitsandbytes produces), a division otherwise.
__device__ __forceinline__ int64_t block_index(const DevWeight &w, int64_t e) {
    return w.bs_shift >= 0 ? (e >> w.bs_shift) : e / w.blocksize;
}
__device__ __forceinline__ int64_t group_index(const DevWeight &w, int64_t b) {
    return w.bs2_shift >= 0 ? (b >> w.bs2_shift) : b / w.blocksize2;
}

// The fp32 absmax of block b: fp32(code2[q] * absmax2[b / blocksize2]) + offset, each operation
// rounded on its own (no fused multiply-add), or the stored fp32 value when not nested.
__device__ __forceinline__ float absmax_of(const DevWeight &w, const float *code2_lds, int64_t b) {
    if (w.nested) {
        const uint8_t q = static_cast<const uint8_t *>(w.absmax)[b];
        const float s = w.absmax2[group_index(w, b)];
        return __fadd_rn(__fmul_rn(code2_lds[q], s), w.offset);
    }
    return static_cast<const float *>(w.absmax)[b];
}

// Two fp32 values rounded to nearest-even into a packed pair (v_cvt_pk_f16_f32 /
// v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack2_f16(float a, float b) {
    half2_t h = __builtin_convertvector((float2_t){a, b}, half2_t);
    return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
    bf162_t h = __builtin_convertvector((float2_t){a, b}, bf162_t);
    return __builtin_bit_cast(uint32_t, h);
}
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (DT == NF4_BF16) return pack2_bf16(a, b);
    else return pack2_f16(a, b);
}

// One fp32 value rounded to nearest-even into fp16 / bf16 bits.  The empty asm keeps the fp32
// value itself as the conversion's input: otherwise a product followed by the conversion can
// be merged into one mixed-precision FMA (v_fma_mixlo_f16), which rounds the exact product once
// instead of rounding the fp32 product, and differs where that fp32 product is an exact tie
// between two fp16 values.
template <int DT>
__device__ __forceinline__ uint16_t round16(float v) {
    asm volatile("" : "+v"(v));
    if constexpr (DT == NF4_BF16) return __builtin_bit_cast(uint16_t, static_cast<bf16_t>(v));
    else return __builtin_bit_cast(uint16_t, static_cast<half_t>(v));
}

// ---------------------------------------------------------- register-table NF4 lookup
//
// For one absmax s, the 16 possible dequantized values round(code[i] * s) (each the same single
// fp32 product and single RNE rounding as the element-wise formula) are packed into byte planes:
// lo[k] holds the low bytes of entries 4k..4k+3, hi[k] their high bytes.  v_perm_b32 then picks
// 4 entries at once by nibble: two perms select within entries 0-7 and 8-15, a third chooses
// between them by bit 3 of each nibble, and two more interleave low and high bytes into
// 16-bit pairs.  No LDS access and no latency chain.

static constexpr uint32_t kPermLoBytes = 0x06040200u;  // bytes 0,2 of S1 and of S0
static constexpr uint32_t kPermHiBytes = 0x07050301u;  // bytes 1,3 of S1 and of S0

struct Nf4Table {
    uint32_t lo[4];
    uint32_t hi[4];
};

__device__ __forceinline__ uint32_t vperm(uint32_t s0, uint32_t s1, uint32_t sel) {
    return __builtin_amdgcn_perm(s0, s1, sel);
}

template <int DT>
__device__ __forceinline__ Nf4Table make_table(const float (&code)[16], float s) {
    uint32_t t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = pack2<DT>(__fmul_rn(code[2 * j], s), __fmul_rn(code[2 * j + 1], s));
    Nf4Table r;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        r.lo[k] = vperm(t[2 * k + 1], t[2 * k], kPermLoBytes);
        r.hi[k] = vperm(t[2 * k + 1], t[2 * k], kPermHiBytes);
    }
    return r;
}

// Half tables.  Where the two lanes of a pair (lane, lane ^ 1) dequantize the same absmax block,
// lane h of the pair forms the entries 8h .. 8h + 7 of the block's table and receives the other
// eight from its partner by a DPP swap: 8 products, 4 conversions, 4 perms and 4 swaps per lane
// instead of 16, 8 and 8.  Slots 0-1 hold the lane's own half and slots 2-3 its partner's, so
// on the odd lane the entry of nibble n sits where the full table keeps n ^ 8: its lookups flip
// bit 3 through the selector base (lookup4s).
struct Nf4HalfCodes {
    float c[8];        // code[8h + i]
    uint32_t selbase;  // byte i: i (even lane) or 4 + i (odd lane)
};

__device__ __forceinline__ Nf4HalfCodes half_codes(const float (&code)[16]) {
    const bool odd = (threadIdx.x & 1) != 0;
    Nf4HalfCodes h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h.c[i] = odd ? code[8 + i] : code[i];
    h.selbase = odd ? 0x07060504u : 0x03020100u;
    return h;
}

// v from lane ^ 1 (quad_perm [1, 0, 3, 2])
__device__ __forceinline__ uint32_t swap_pair(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xB1, 0xF, 0xF, true));
}

template <int DT>
__device__ __forceinline__ Nf4Table make_table_half(const Nf4HalfCodes &hc, float s) {
    uint32_t t[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) t[j] = pack2<DT>(__fmul_rn(hc.c[2 * j], s), __fmul_rn(hc.c[2 * j + 1], s));
    Nf4Table r;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        r.lo[k] = vperm(t[2 * k + 1], t[2 * k], kPermLoBytes);
        r.hi[k] = vperm(t[2 * k + 1], t[2 * k], kPermHiBytes);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        r.lo[2 + k] = swap_pair(r.lo[k]);
        r.hi[2 + k] = swap_pair(r.hi[k]);
    }
    return r;
}

// The same for the pair (lane, lane ^ 16), the partner's half through the LDS crossbar
// (ds_swizzle, xor mask 16 within each 32 lanes; no LDS memory): lane bit 4 picks the half.
__device__ __forceinline__ Nf4HalfCodes half_codes16(const float (&code)[16]) {
    const bool odd = (threadIdx.x & 16) != 0;
    Nf4HalfCodes h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h.c[i] = odd ? code[8 + i] : code[i];
    h.selbase = odd ? 0x07060504u : 0x03020100u;
    return h;
}

__device__ __forceinline__ uint32_t swap_lane16(uint32_t v) {
    // bit mode: and 0x1f, or 0, xor 0x10
    return static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v), 0x401F));
}

template <int DT>
__device__ __forceinline__ Nf4Table make_table_half16(const Nf4HalfCodes &hc, float s) {
    uint32_t t[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) t[j] = pack2<DT>(__fmul_rn(hc.c[2 * j], s), __fmul_rn(hc.c[2 * j + 1], s));
    Nf4Table r;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        r.lo[k] = vperm(t[2 * k + 1], t[2 * k], kPermLoBytes);
        r.hi[k] = vperm(t[2 * k + 1], t[2 * k], kPermHiBytes);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        r.lo[2 + k] = swap_lane16(r.lo[k]);
        r.hi[2 + k] = swap_lane16(r.hi[k]);
    }
    return r;
}

// 8 elements of a packed dword in nibble-plane order (lookup8_planes) through a half table.
__device__ __forceinline__ u32x4_t lookup8_planes_s(const Nf4Table &t, uint32_t p, uint32_t selbase);

// 4 nibbles s (one per byte, element order) -> 4 table entries as two packed pairs; `selbase`
// picks the half of the table that bit 3 of a nibble selects (0x03020100 for a full table).
__device__ __forceinline__ void lookup4s(const Nf4Table &t, uint32_t s, uint32_t selbase,
                                         uint32_t &o0, uint32_t &o1) {
    const uint32_t s7 = s & 0x07070707u;
    const uint32_t sel = ((s >> 1) & 0x04040404u) ^ selbase;  // one v_bitop3
    const uint32_t lo = vperm(vperm(t.lo[3], t.lo[2], s7), vperm(t.lo[1], t.lo[0], s7), sel);
    const uint32_t hi = vperm(vperm(t.hi[3], t.hi[2], s7), vperm(t.hi[1], t.hi[0], s7), sel);
    o0 = vperm(hi, lo, 0x05010400u);
    o1 = vperm(hi, lo, 0x07030602u);
}

// The 8 elements of one packed dword through a half table (lookup8 below, selector base of
// the lane's half).
__device__ __forceinline__ u32x4_t lookup8s(const Nf4Table &t, uint32_t p, uint32_t selbase) {
    const uint32_t hi4 = (p >> 4) & 0x0F0F0F0Fu;
    const uint32_t lo4 = p & 0x0F0F0F0Fu;
    uint32_t o0, o1, o2, o3;
    lookup4s(t, vperm(lo4, hi4, 0x05010400u), selbase, o0, o1);
    lookup4s(t, vperm(lo4, hi4, 0x07030602u), selbase, o2, o3);
    return (u32x4_t){o0, o1, o2, o3};
}

// 4 nibbles s (one per byte, element order) -> 4 table entries as two packed pairs.
__device__ __forceinline__ void lookup4(const Nf4Table &t, uint32_t s, uint32_t &o0, uint32_t &o1) {
    const uint32_t s7 = s & 0x07070707u;
    const uint32_t sel = ((s >> 1) & 0x04040404u) | 0x03020100u;  // byte i: i, or 4 + i if bit 3
    const uint32_t lo = vperm(vperm(t.lo[3], t.lo[2], s7), vperm(t.lo[1], t.lo[0], s7), sel);
    const uint32_t hi = vperm(vperm(t.hi[3], t.hi[2], s7), vperm(t.hi[1], t.hi[0], s7), sel);
    o0 = vperm(hi, lo, 0x05010400u);
    o1 = vperm(hi, lo, 0x07030602u);
}

// The 8 elements of one packed dword (byte j: high nibble = element 2j, low = 2j+1), as four
// packed 16-bit pairs in element order.
__device__ __forceinline__ u32x4_t lookup8(const Nf4Table &t, uint32_t p) {
    const uint32_t hi4 = (p >> 4) & 0x0F0F0F0Fu;   // byte j: element 2j
    const uint32_t lo4 = p & 0x0F0F0F0Fu;          // byte j: element 2j + 1
    uint32_t o0, o1, o2, o3;
    lookup4(t, vperm(lo4, hi4, 0x05010400u), o0, o1);  // elements 0..3
    lookup4(t, vperm(lo4, hi4, 0x07030602u), o2, o3);  // elements 4..7
    return (u32x4_t){o0, o1, o2, o3};
}

// The same 8 elements in nibble-plane order: the high nibbles' entries, then the low nibbles'
// (elements 0, 2, 4, 6, 1, 3, 5, 7 as four packed pairs).  An MFMA reduction is indifferent to
// the order of its k values as long as both operands use the same one: the other operand's 8
// values go through `plane_order` once, which saves the two perms that restore element order.
__device__ __forceinline__ u32x4_t lookup8_planes(const Nf4Table &t, uint32_t p) {
    uint32_t o0, o1, o2, o3;
    lookup4(t, (p >> 4) & 0x0F0F0F0Fu, o0, o1);
    lookup4(t, p & 0x0F0F0F0Fu, o2, o3);
    return (u32x4_t){o0, o1, o2, o3};
}

__device__ __forceinline__ u32x4_t lookup8_planes_s(const Nf4Table &t, uint32_t p, uint32_t selbase) {
    uint32_t o0, o1, o2, o3;
    lookup4s(t, (p >> 4) & 0x0F0F0F0Fu, selbase, o0, o1);
    lookup4s(t, p & 0x0F0F0F0Fu, selbase, o2, o3);
    return (u32x4_t){o0, o1, o2, o3};
}

// 8 consecutive 16-bit values (x0 .. x7 as four packed pairs) in the order of lookup8_planes.
__device__ __forceinline__ u32x4_t plane_order(u32x4_t c) {
    return (u32x4_t){vperm(c.y, c.x, 0x05040100u), vperm(c.w, c.z, 0x05040100u),
                     vperm(c.y, c.x, 0x07060302u), vperm(c.w, c.z, 0x07060302u)};
}

// The NF4 table of a weight in scalar registers (the same for every lane).
__device__ __forceinline__ void load_code_sgpr(const float *code, float (&out)[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
        out[i] = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, code[i])));
}

// ------------------------------------------------------- wave sums and dot products

template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                     CTRL, 0xF, 0xF, false));
}

// Sum of v over the 64 lanes, the same value in every lane, in a fixed order.
__device__ __forceinline__ float wave_sum(float v) {
    v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141>(v);  // row_half_mirror: the two quads of each half row
    v = dpp_add<0x140>(v);  // row_mirror: the two halves of each row
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    if constexpr (DT == NF4_BF16)
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162_t, a),
                                               __builtin_bit_cast(bf162_t, b), c, false);
    else
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b),
                                      c, false);
}

// ----------------------------------------------------------------- buffer resources
//
// Main-loop loads go through buffer resources: an offset at or past the resource's byte range
// returns zero in hardware.  Every lane then issues the same unconditional loads (no divergent
// branches in the pipeline, so the compiler's wait counters stay exact), rows past M and weight
// rows past the segment read as zero, and nothing outside an operand is ever touched.

typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, int64_t bytes) {
    const int n = bytes > 0x7fffffff ? 0x7fffffff : (bytes < 0 ? 0 : static_cast<int>(bytes));
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), n,
                                             0x00020000);
}
__device__ __forceinline__ u32x4_t bload16(rsrc_t r, int off) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t bload4(rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t bload2(rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t bload1(rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
}

static inline int status_of(hipError_t e) { return e == hipSuccess ? NF4_OK : NF4_ERR_LAUNCH; }

static inline bool aligned(const void *p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

static inline int dtype_bytes(int dt) { return dt == NF4_F32 ? 4 : 2; }

// Validates one weight descriptor; returns NF4_OK or an error status.
static inline int check_weight(const nf4_weight *w) {
    if (!w) return NF4_ERR_ARG;
    if (w->rows < 0 || w->cols < 0 || w->blocksize <= 0 || (w->blocksize & 1)) return NF4_ERR_ARG;
    if (w->rows == 0 || w->cols == 0) return NF4_OK;  // empty: nothing is read
    if (!w->packed || !w->absmax || !w->code) return NF4_ERR_ARG;
    if (w->nested) {
        if (!w->absmax2 || !w->code2 || w->blocksize2 <= 0) return NF4_ERR_ARG;
    }
    return NF4_OK;
}
