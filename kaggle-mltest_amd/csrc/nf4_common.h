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
};

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
    return d;
}

// The fp32 absmax of block b: fp32(code2[q] * absmax2[b / blocksize2]) + offset, each operation
// rounded on its own (no fused multiply-add), or the stored fp32 value when not nested.
__device__ __forceinline__ float absmax_of(const DevWeight &w, const float *code2_lds, int64_t b) {
    if (w.nested) {
        const uint8_t q = static_cast<const uint8_t *>(w.absmax)[b];
        const float s = w.absmax2[b / w.blocksize2];
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
