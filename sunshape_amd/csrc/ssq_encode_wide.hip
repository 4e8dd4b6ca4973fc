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
// have a strictly smaller distance, and only new minima take a sqrt.  The first index reaching the
// final minimum distance was a new minimum when it was reached (every earlier index has a larger
// distance, hence a larger pre-sqrt value), and a later index with an equal distance does not
// replace it (strict comparison).
#include "ssq_encode_math.h"

#include <math.h>

namespace {

constexpr int kWideThreads = 256;
constexpr int kWideStageFloats = 16384;  // 64 KiB per LDS stage: chunk * (bd + 1) floats

struct WideEncodeParams {
    ssq_encode_args a;
    int fold;   // short sequences: all sequences of a KV head share one key range (SsqKeyMap)
    int chunk;  // codewords per LDS stage
};

__device__ __forceinline__ void store_code(uint8_t* codes, int width, int64_t i, uint32_t v) {
    if (width == 2) reinterpret_cast<uint16_t*>(codes)[i] = (uint16_t)v;
    else reinterpret_cast<uint32_t*>(codes)[i] = v;
}

__global__ __launch_bounds__(kWideThreads) void k_encode_wide(const WideEncodeParams p) {
    extern __shared__ __align__(16) float smem[];
    const ssq_encode_args& a = p.a;
    const SsqKeyMap km(a, p.fold);
    const int kv = km.kv;
    const int blk = blockIdx.z;
    const int bd = a.block_dim, nc = a.n_centroids, D = a.head_dim;
    const int cw = ssq_code_width(nc);
    const bool heavy = ssq_is_heavy(a.heavy_mask[0], a.heavy_mask[1], blk);  // uniform per workgroup
    const int i = blockIdx.x * kWideThreads + threadIdx.x;
    const bool live = i < km.n_keys;
    const float* met = a.metric ? a.metric + (int64_t)kv * a.metric_sh + (int64_t)blk * bd * D + blk * bd : nullptr;
    float x[16];
    int64_t crow = 0, prow = 0;
    if (live) {
        int b, s;
        km.bs(a, i, b, s);
        const int64_t kbase = (int64_t)b * a.k_sb + (int64_t)kv * a.k_sh + (int64_t)s * a.k_ss;
        const int64_t* perm = a.perm + (int64_t)kv * a.perm_sh + blk * bd;
        for (int d = 0; d < bd; ++d) x[d] = ssq_load_elem(a.keys, a.k_dtype, kbase + perm[d]);
        out_rows(a, b, kv, s, crow, prow);
        if (heavy) {  // passthrough block: code 0, values copied (sunshape/codec.py:367-372)
            store_code(a.codes, cw, crow + blk, 0u);
            const int slot = a.pt_dense ? blk : heavy_ordinal(a.heavy_mask[0], a.heavy_mask[1], blk);
            for (int d = 0; d < bd; ++d) ssq_store_elem(a.pt, a.pt_dtype, prow + (int64_t)slot * bd + d, x[d]);
        } else if (met) {
            float y[16];
            for (int k = 0; k < bd; ++k) y[k] = metric_row(met + (int64_t)k * D, x, bd);
            for (int k = 0; k < bd; ++k) x[k] = y[k];
        }
    }
    if (heavy) return;  // the whole workgroup: no barrier follows for it
    const float xn = sq_norm(x, bd);
    const bool direct = a.direct_dist != 0;
    float* cb = smem;                          // [chunk][bd]
    float* cn = smem + (size_t)p.chunk * bd;   // [chunk]
    const float* cent = a.cent + (int64_t)kv * a.cent_sh + (int64_t)blk * nc * bd;
    float e_min = INFINITY, f_best = INFINITY;
    uint32_t j_best = 0;
    for (int j0 = 0; j0 < nc; j0 += p.chunk) {
        const int n = min(p.chunk, nc - j0);
        __syncthreads();  // the previous chunk's reads are done
        for (int e = threadIdx.x; e < n; e += kWideThreads) {
            const float* c = cent + (int64_t)(j0 + e) * bd;
            float cv[16];
            for (int d = 0; d < bd; ++d) cv[d] = c[d];
            if (met) {
                float y[16];
                for (int k = 0; k < bd; ++k) y[k] = metric_row(met + (int64_t)k * D, cv, bd);
                for (int k = 0; k < bd; ++k) cv[k] = y[k];
            }
            for (int d = 0; d < bd; ++d) cb[(size_t)e * bd + d] = cv[d];
            cn[e] = sq_norm(cv, bd);
        }
        __syncthreads();
        if (live) {
            for (int j = 0; j < n; ++j) {
                const float* c = cb + (size_t)j * bd;
                // clamped as the reference's sqrt(clamp_min(., 0)): NaN (a non-finite key) is 0
                const float v = direct ? direct_dist2(x, c, bd) : mm_dist2(x, xn, c, cn[j], bd);
                const float vc = v > 0.f ? v : 0.f;
                if (vc < e_min) {
                    e_min = vc;
                    const float f = dist_of(v);
                    if (f < f_best) {
                        f_best = f;
                        j_best = (uint32_t)(j0 + j);
                    }
                }
            }
        }
    }
    if (live) store_code(a.codes, cw, crow + blk, j_best);
}

}  // namespace

int ssq_encode_wide_run(const ssq_encode_args* a, hipStream_t st) {
    WideEncodeParams p;
    p.a = *a;
    const int stage = kWideStageFloats / (a->block_dim + 1);
    p.chunk = a->n_centroids < stage ? a->n_centroids : stage;
    p.fold = ssq_encode_fold(a, kWideThreads);
    const int64_t n_keys = p.fold ? (int64_t)a->batch * a->seq_len : a->seq_len;
    dim3 grid((unsigned)((n_keys + kWideThreads - 1) / kWideThreads), p.fold ? a->num_kv_heads : a->batch * a->num_kv_heads,
              a->n_blocks);
    const size_t smem = (size_t)p.chunk * (a->block_dim + 1) * sizeof(float);
    hipLaunchKernelGGL(k_encode_wide, grid, dim3(kWideThreads), smem, st, p);
    return ssq_check_hip(hipGetLastError(), "k_encode_wide launch");
}
