// The reference's distance arithmetic for the encode kernels (ssq_encode.hip, ssq_encode_wide.hip):
// torch.cdist's mm formulation and direct evaluation, the SunShape-Pro block metric, and the output
// addressing shared by the kernels.  Sources including it are compiled with -ffp-contract=off, so
// every multiply-add that is not an explicit fmaf stays two roundings.
#pragma once

#include "ssq_common.h"

namespace {

// |v|^2 as x.pow(2).sum(-1): squares rounded, summed left to right (no contraction)
__device__ __forceinline__ float sq_norm(const float* v, int bd) {
    float s = v[0] * v[0];
    for (int d = 1; d < bd; ++d) {
        const float t = v[d] * v[d];
        s = s + t;
    }
    return s;
}

// pre-sqrt distance: k ascending FMA chain over [-2x, xn, 1] . [c, 1, cn]
__device__ __forceinline__ float mm_dist2(const float* x, float xn, const float* c, float cn, int bd) {
    float acc = (-2.0f * x[0]) * c[0];
    for (int d = 1; d < bd; ++d) acc = __builtin_fmaf(-2.0f * x[d], c[d], acc);
    acc = __builtin_fmaf(xn, 1.0f, acc);
    acc = __builtin_fmaf(1.0f, cn, acc);
    return acc;
}

// y_k = sum_j e[k*ld + j] * x[j] for one row k of a SunShape-Pro block metric E_b:
// j ascending, first product rounded, then fused multiply-adds
__device__ __forceinline__ float metric_row(const float* e, const float* x, int bd) {
    float acc = e[0] * x[0];
    for (int j = 1; j < bd; ++j) acc = __builtin_fmaf(e[j], x[j], acc);
    return acc;
}

// pre-sqrt distance of torch.cdist's direct evaluation (the one it takes when both inputs have at
// most 25 rows): sum over k ascending of the rounded squares (x_k - c_k)^2, summed left to right
__device__ __forceinline__ float direct_dist2(const float* x, const float* c, int bd) {
    float d = x[0] - c[0];
    float s = d * d;
    for (int k = 1; k < bd; ++k) {
        d = x[k] - c[k];
        const float t = d * d;
        s = s + t;
    }
    return s;
}

// correctly rounded sqrt of max(v, 0)
__device__ __forceinline__ float dist_of(float v) { return __builtin_sqrtf(v > 0.f ? v : 0.f); }

__device__ __forceinline__ int heavy_ordinal(uint64_t hm0, uint64_t hm1, int blk) {
    if (blk < 64) return __popcll(hm0 & ((1ull << blk) - 1ull));
    return __popcll(hm0) + __popcll(hm1 & ((1ull << (blk - 64)) - 1ull));
}

// output row bases for key (b, kv, s): codes and passthrough
__device__ __forceinline__ void out_rows(const ssq_encode_args& a, int b, int kv, int s, int64_t& crow,
                                         int64_t& prow) {
    if (a.slot_mapping) {
        const int64_t slot = a.slot_mapping[(int64_t)b * a.sm_sb + s];
        const int64_t page = slot / a.page_size, off = slot - page * a.page_size;
        crow = page * a.c_sb + (int64_t)kv * a.c_sh + off * a.c_st;
        prow = page * a.pt_sb + (int64_t)kv * a.pt_sh + off * a.pt_st;
    } else {
        crow = (int64_t)b * a.c_sb + (int64_t)kv * a.c_sh + (int64_t)s * a.c_st;
        prow = (int64_t)b * a.pt_sb + (int64_t)kv * a.pt_sh + (int64_t)s * a.pt_st;
    }
}

}  // namespace
