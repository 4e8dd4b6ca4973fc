// Nearest-codeword encode for codebooks of more than 256 codewords: 16-bit codes up to 65535
// codewords, 32-bit beyond, as the reference's _compact_index_dtype stores them
// (sunshape/codec.py:78-83; SunShapeBlockCodec.quantize, :362-385).  The reference's default
// fitter gives such codebooks at bits_per_dim * block_dim > 8 (n_centroids = 2^round(bits * bd),
// sunshape/hf.py:594): 4,096 codewords at 3 bits/dim and block_dim 4.
//
// One thread per (key, block), one light block per workgroup (blockIdx.z); the block's codewords
// pass through LDS in chunks (in the metric space E_b c under a SunShape-Pro metric) with their
// norms.  The index is the first argmin of the reference's fp32 distance, sqrt(max(d2, 0)) with d2
// in torch.cdist's mm formulation (or its direct one), in one pass: a correctly rounded sqrt is
// non-decreasing, so a codeword whose pre-sqrt value is not below the smallest seen so far cannot
// have a strictly smaller distance, and only new pre-sqrt minima are examined further (take_min).
// The first index reaching the final minimum distance was a new minimum when it was reached (every
// earlier index has a larger distance, hence a larger pre-sqrt value), and a later index with an
// equal distance does not replace it (strict comparison).
#include "ssq_encode_math.h"

#include <math.h>

namespace {

constexpr int kWideThreads = 256;
constexpr int kWideStageFloats = 4096;  // 16 KiB per LDS stage: chunk * (bd + 1) floats

struct WideEncodeParams {
    ssq_encode_args a;
    int fold;     // short sequences: all sequences of a KV head share one key range (SsqKeyMap)
    int chunk;    // codewords per LDS stage
    int slices;   // lanes per (key, block), a power of two <= 64: lane s scans codewords s, s + slices, ...
    int vec;      // 1: each codeword row is 4 * block_dim-byte aligned (vector staging loads)
};

__device__ __forceinline__ void store_code(uint8_t* codes, int width, int64_t i, uint32_t v) {
    if (width == 2) reinterpret_cast<uint16_t*>(codes)[i] = (uint16_t)v;
    else reinterpret_cast<uint32_t*>(codes)[i] = v;
}

// one codeword's pre-sqrt distance v (not yet clamped)
template <int BD, bool MM>
__device__ __forceinline__ float stage_dist(const float* x, float xn, const float* cb, const float* cn, int j, int bd) {
    const int w = BD ? BD : bd;
    const float* c = cb + (size_t)j * w;
    return MM ? mm_dist2(x, xn, c, cn[j], w) : direct_dist2(x, c, w);
}

// A codeword's pre-sqrt value v, clamped as the reference's sqrt(clamp_min(., 0)) clamps it (NaN
// and negatives: 0), against the smallest clamped value so far, e_min >= 0.  The common test,
// !(v >= e_min), holds whenever the clamped value is below e_min (v < e_min, or v NaN, or v <= 0
// while e_min > 0); the clamp and the exact test follow only then.  New minima are rare after a
// lane's first codewords, and the empty volatile asm statements keep these branches, so that
// nothing past the common test is evaluated for every codeword.  The index moves when the new
// value's correctly rounded sqrt is below e_min's.  A correctly rounded sqrt merges
// pre-sqrt values less than 2^-21 apart relatively at most (below 2^-126, a few units of the
// smallest subnormal), so a value below t = e_min (1 - 2^-20) - 2^-146 has the smaller sqrt;
// between t and e_min the two sqrts are compared.
__device__ __forceinline__ void take_min(float v, uint32_t j, float& e_min, uint32_t& j_best) {
    if (!(v >= e_min)) {
        __asm__ volatile("");
        const float vc = v > 0.f ? v : 0.f;
        if (!(vc < e_min)) return;
        const float t = e_min * 0x1.ffffep-1f - 0x1.0p-146f;
        if (vc < t) {
            j_best = j;
        } else {
            __asm__ volatile("");
            if (__builtin_sqrtf(vc) < __builtin_sqrtf(e_min)) j_best = j;
        }
        e_min = vc;
    }
}

// one LDS stage's codewords sl, sl + S, ... < n (ONE: S == 1) in ascending order; with the block
// dim known, eight codewords' distances are computed before their minimum checks, so that their
// LDS reads are in flight together
template <int BD, bool MM, bool ONE>
__device__ __forceinline__ void scan_stage(const float* x, float xn, const float* cb, const float* cn, int bd, int sl,
                                           int S, int n, int j0, float& e_min, uint32_t& j_best) {
    const int st = ONE ? 1 : S;
    int j = ONE ? 0 : sl;
    if (BD) {
        for (; j + 7 * st < n; j += 8 * st) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = stage_dist<BD, MM>(x, xn, cb, cn, j + u * st, bd);
#pragma unroll
            for (int u = 0; u < 8; ++u) take_min(v[u], (uint32_t)(j0 + j + u * st), e_min, j_best);
        }
    }
    for (; j < n; j += st) take_min(stage_dist<BD, MM>(x, xn, cb, cn, j, bd), (uint32_t)(j0 + j), e_min, j_best);
}

// BD: the block dim at compile time (1, 2, 4 or 8), or 0 for any other (read from the arguments).
// A workgroup serves kWideThreads / slices keys of one block; the slices lanes of a key sit next
// to each other in a wave and split the codebook between them (lane s takes codewords s,
// s + slices, ... in ascending order), each finding the first minimum of its own codewords; the
// lanes then combine (smaller distance, then smaller index), which gives the first argmin over
// the whole codebook.
template <int BD>
__global__ __launch_bounds__(kWideThreads) void k_encode_wide(const WideEncodeParams p) {
    extern __shared__ __align__(16) float smem[];
    const ssq_encode_args& a = p.a;
    const SsqKeyMap km(a, p.fold);
    const int kv = km.kv;
    const int blk = blockIdx.z;
    const int bd = BD ? BD : a.block_dim, nc = a.n_centroids, D = a.head_dim;
    constexpr int kX = BD ? BD : 16;
    const int cw = ssq_code_width(nc);
    const bool heavy = ssq_is_heavy(a.heavy_mask[0], a.heavy_mask[1], blk);  // uniform per workgroup
    const int S = p.slices;
    const int sl = threadIdx.x & (S - 1);
    const int i = blockIdx.x * (kWideThreads / S) + (int)(threadIdx.x / S);
    const bool live = i < km.n_keys;
    const float* met = a.metric ? a.metric + (int64_t)kv * a.metric_sh + (int64_t)blk * bd * D + blk * bd : nullptr;
    float x[kX];
    int64_t crow = 0, prow = 0;
    if (live) {
        int b, s;
        km.bs(a, i, b, s);
        const int64_t kbase = (int64_t)b * a.k_sb + (int64_t)kv * a.k_sh + (int64_t)s * a.k_ss;
        const int64_t* perm = a.perm + (int64_t)kv * a.perm_sh + blk * bd;
#pragma unroll
        for (int d = 0; d < kX; ++d)
            if (d < bd) x[d] = ssq_load_elem(a.keys, a.k_dtype, kbase + perm[d]);
        out_rows(a, b, kv, s, crow, prow);
        if (heavy) {  // passthrough block: code 0, values copied (sunshape/codec.py:367-372)
            if (sl == 0) {
                store_code(a.codes, cw, crow + blk, 0u);
                const int slot = a.pt_dense ? blk : heavy_ordinal(a.heavy_mask[0], a.heavy_mask[1], blk);
                for (int d = 0; d < bd; ++d) ssq_store_elem(a.pt, a.pt_dtype, prow + (int64_t)slot * bd + d, x[d]);
            }
        } else if (met) {
            float y[kX];
#pragma unroll
            for (int k = 0; k < kX; ++k)
                if (k < bd) y[k] = metric_row(met + (int64_t)k * D, x, bd);
#pragma unroll
            for (int k = 0; k < kX; ++k)
                if (k < bd) x[k] = y[k];
        }
    }
    if (heavy) return;  // the whole workgroup: no barrier follows for it
    const float xn = sq_norm(x, bd);
    const bool direct = a.direct_dist != 0;
    float* cb = smem;                          // [chunk][bd]
    float* cn = smem + (size_t)p.chunk * bd;   // [chunk]
    const float* cent = a.cent + (int64_t)kv * a.cent_sh + (int64_t)blk * nc * bd;
    float e_min = INFINITY;  // the smallest clamped pre-sqrt value; its sqrt is the lane's distance
    uint32_t j_best = 0;
    for (int j0 = 0; j0 < nc; j0 += p.chunk) {
        const int n = min(p.chunk, nc - j0);
        __syncthreads();  // the previous chunk's reads are done
        for (int e = threadIdx.x; e < n; e += kWideThreads) {
            const float* c = cent + (int64_t)(j0 + e) * bd;
            float cv[kX];
            if (BD == 4 && p.vec) {
                const float4 v = *reinterpret_cast<const float4*>(c);
                cv[0] = v.x; cv[1] = v.y; cv[2] = v.z; cv[3] = v.w;
            } else if (BD == 2 && p.vec) {
                const float2 v = *reinterpret_cast<const float2*>(c);
                cv[0] = v.x; cv[1] = v.y;
            } else {
#pragma unroll
                for (int d = 0; d < kX; ++d)
                    if (d < bd) cv[d] = c[d];
            }
            if (met) {
                float y[kX];
#pragma unroll
                for (int k = 0; k < kX; ++k)
                    if (k < bd) y[k] = metric_row(met + (int64_t)k * D, cv, bd);
#pragma unroll
                for (int k = 0; k < kX; ++k)
                    if (k < bd) cv[k] = y[k];
            }
#pragma unroll
            for (int d = 0; d < kX; ++d)
                if (d < bd) cb[(size_t)e * bd + d] = cv[d];
            cn[e] = sq_norm(cv, bd);
        }
        __syncthreads();
        if (live) {
            if (S == 1) {
                if (direct) scan_stage<BD, false, true>(x, xn, cb, cn, bd, sl, S, n, j0, e_min, j_best);
                else scan_stage<BD, true, true>(x, xn, cb, cn, bd, sl, S, n, j0, e_min, j_best);
            } else {
                if (direct) scan_stage<BD, false, false>(x, xn, cb, cn, bd, sl, S, n, j0, e_min, j_best);
                else scan_stage<BD, true, false>(x, xn, cb, cn, bd, sl, S, n, j0, e_min, j_best);
            }
        }
    }
    // combine the key's lanes: the smaller distance, then the smaller index (every lane of a
    // workgroup reaches this point; lanes of keys past the end carry infinities and are not stored)
    float f_best = __builtin_sqrtf(e_min);
    for (int o = S >> 1; o > 0; o >>= 1) {
        const float of = __shfl_xor(f_best, o);
        const uint32_t oj = (uint32_t)__shfl_xor((int)j_best, o);
        if (of < f_best || (of == f_best && oj < j_best)) {
            f_best = of;
            j_best = oj;
        }
    }
    if (live && sl == 0) store_code(a.codes, cw, crow + blk, j_best);
}

}  // namespace

int ssq_encode_wide_run(const ssq_encode_args* a, hipStream_t st) {
    WideEncodeParams p;
    p.a = *a;
    const int stage = kWideStageFloats / (a->block_dim + 1);
    p.chunk = a->n_centroids < stage ? a->n_centroids : stage;
    p.fold = ssq_encode_fold(a, kWideThreads);
    const int64_t n_keys = p.fold ? (int64_t)a->batch * a->seq_len : a->seq_len;
    const int64_t units = n_keys * (p.fold ? a->num_kv_heads : (int64_t)a->batch * a->num_kv_heads) * a->n_blocks;
    // a launch with few (key, block) pairs (a decode step's append) splits each codebook scan over
    // several lanes, up to about 2^18 lanes in all, and at least 16 codewords per lane
    p.slices = 1;
    while (p.slices < 64 && units * p.slices < (1 << 18) && p.slices * 16 <= a->n_centroids) p.slices *= 2;
    const int bd = a->block_dim;
    const int64_t row_bytes = (int64_t)bd * 4;
    p.vec = ((uintptr_t)a->cent % (bd == 4 ? 16 : 8) == 0 && (a->cent_sh * 4) % (bd == 4 ? 16 : 8) == 0 &&
             ((int64_t)a->n_centroids * row_bytes) % (bd == 4 ? 16 : 8) == 0) ? 1 : 0;
    const int keys_wg = kWideThreads / p.slices;
    dim3 grid((unsigned)((n_keys + keys_wg - 1) / keys_wg), p.fold ? a->num_kv_heads : a->batch * a->num_kv_heads,
              a->n_blocks);
    const size_t smem = (size_t)p.chunk * (bd + 1) * sizeof(float);
    switch (bd) {
        case 1: hipLaunchKernelGGL(k_encode_wide<1>, grid, dim3(kWideThreads), smem, st, p); break;
        case 2: hipLaunchKernelGGL(k_encode_wide<2>, grid, dim3(kWideThreads), smem, st, p); break;
        case 4: hipLaunchKernelGGL(k_encode_wide<4>, grid, dim3(kWideThreads), smem, st, p); break;
        case 8: hipLaunchKernelGGL(k_encode_wide<8>, grid, dim3(kWideThreads), smem, st, p); break;
        default: hipLaunchKernelGGL(k_encode_wide<0>, grid, dim3(kWideThreads), smem, st, p); break;
    }
    return ssq_check_hip(hipGetLastError(), "k_encode_wide launch");
}
