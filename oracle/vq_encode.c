/*
 * CPU restatement of SunShape's nearest-codeword encode -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker.  The product path never calls it.
 *
 * Follows sunshape/codec.py:362-385 (SunShapeBlockCodec.quantize):
 *   keys.float() -> x[..., perm] -> per block b:
 *     heavy (mixed mode): passthrough_values[:, b, :] = x_b, index 0
 *     else: argmin_c torch.cdist(x_b @ E_b^T, C_b @ E_b^T)
 *           E_b = E[b*bd:(b+1)*bd, b*bd:(b+1)*bd], the block's diagonal block of the
 *           [D, D] metric (identity outside SunShape-Pro, sunshape/codec.py:289-312).
 *           y = x_b @ E_b^T is evaluated row by row as y_k = sum_j E_b[k][j] * x_j with
 *           j ascending, first product rounded, then fused multiply-adds; C_b @ E_b^T
 *           likewise.  (torch's matmul leaves its order unspecified; this is the
 *           order the HIP kernels use, and an identity E reproduces x exactly.)
 * torch.cdist with >25 rows takes ATen's mm formulation (_euclidean_dist):
 *   x1_ = [-2*x, |x|^2, 1],  x2_ = [c, 1, |c|^2],  d2 = x1_ @ x2_^T,
 *   d = sqrt(clamp_min(d2, 0)),  argmin -> first minimum.
 * |x|^2 is x.pow(2).sum(-1): each square rounded, summed left to right.
 * The fp32 GEMM with K = bd + 2 accumulates k = 0..K-1 in order with fused
 * multiply-adds, starting from the first product (checked bit-for-bit against
 * torch's CPU matmul in tests/test_oracle_encode.py).
 * sqrt is the correctly rounded IEEE square root (see that test for why).
 * When both of cdist's inputs have at most 25 rows, ATen evaluates the distance directly
 * (the cdist_impl branch that skips _euclidean_dist): sqrt(sum_k (x_k - c_k)^2), each square
 * rounded and summed in k order -- the `direct` flag (checked in tests/test_oracle_encode.py
 * against torch's scalar CPU kernel bit for bit).
 * Rotated mode (sunshape/codec.py:247-259, x @ rotation.T): oracle_transform_rows below.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

/* |v|^2 as x.pow(2).sum(-1): left-to-right sum of rounded squares. */
static float sq_norm(const float* v, int bd) {
    float s = v[0] * v[0];
    for (int d = 1; d < bd; ++d) {
        float t = v[d] * v[d];
        s = s + t;
    }
    return s;
}

/* Pre-sqrt distance of the mm formulation, k ascending, fused multiply-adds. */
static float mm_dist2(const float* x, float xn, const float* c, float cn, int bd) {
    float acc = (-2.0f * x[0]) * c[0];
    for (int d = 1; d < bd; ++d) acc = fmaf(-2.0f * x[d], c[d], acc);
    acc = fmaf(xn, 1.0f, acc);
    acc = fmaf(1.0f, cn, acc);
    return acc;
}

/* Direct pre-sqrt distance: rounded squares of the differences, summed in k order. */
static float direct_dist2(const float* x, const float* c, int bd) {
    float d = x[0] - c[0];
    float s = d * d;
    for (int k = 1; k < bd; ++k) {
        d = x[k] - c[k];
        float t = d * d;
        s = s + t;
    }
    return s;
}

/* y[k] = sum_j e[k*ld + j] * x[j], j ascending, first product rounded, then FMAs. */
static void metric_apply(const float* e, int ld, const float* x, int bd, float* y) {
    for (int k = 0; k < bd; ++k) {
        float acc = e[(int64_t)k * ld] * x[0];
        for (int j = 1; j < bd; ++j) acc = fmaf(e[(int64_t)k * ld + j], x[j], acc);
        y[k] = acc;
    }
}

/* Distance matrix for one block: e2[i*nc+j] = pre-sqrt value, d[i*nc+j] = sqrt(clamp_min(., 0)).
 * direct != 0: the direct evaluation in place of the mm formulation. */
void oracle_block_dist_ex(const float* x, int64_t n, const float* c, int nc, int bd, int direct, float* e2, float* d) {
    for (int64_t i = 0; i < n; ++i) {
        const float* xi = x + i * bd;
        float xn = sq_norm(xi, bd);
        for (int j = 0; j < nc; ++j) {
            const float* cj = c + (int64_t)j * bd;
            float v = direct ? direct_dist2(xi, cj, bd) : mm_dist2(xi, xn, cj, sq_norm(cj, bd), bd);
            if (e2) e2[i * nc + j] = v;
            if (d) d[i * nc + j] = sqrtf(v > 0.0f ? v : 0.0f);
        }
    }
}

void oracle_block_dist(const float* x, int64_t n, const float* c, int nc, int bd, float* e2, float* d) {
    oracle_block_dist_ex(x, n, c, nc, bd, 0, e2, d);
}

/*
 * Encode n keys.
 *   keys      fp32 [n, D] in the original basis (bf16 keys are upcast exactly by the caller)
 *   perm      int64 [D]   forward permutation: x_perm[j] = x[perm[j]]
 *   cent      fp32 [nb, nc, bd] codebook in the permuted basis
 *   heavy     uint8 [nb] or NULL; nonzero = passthrough block (index 0, values copied)
 *   codes     uint8 [n, nb] out
 *   pt        fp32 [n, nb, bd] out or NULL; zeros on light blocks (dense, as the reference)
 */
/*
 * Rows through a dense D x D matrix: out[r, j] = sum_k x[r, k] * m_jk, m_jk = M[j*D + k]
 * (transpose 0: x @ M^T, the rotated mode's _forward_transform) or M[k*D + j] (transpose 1:
 * x @ M, its _inverse_transform); k ascending, the first product rounded, then fused
 * multiply-adds (torch's matmul leaves its order unspecified; this is the order the HIP
 * transform uses).
 */
void oracle_transform_rows(const float* x, int64_t n, int D, const float* M, int transpose, float* out) {
    for (int64_t r = 0; r < n; ++r) {
        const float* xr = x + r * D;
        for (int j = 0; j < D; ++j) {
            float acc = 0.0f;
            for (int k = 0; k < D; ++k) {
                const float m = transpose ? M[(int64_t)k * D + j] : M[(int64_t)j * D + k];
                acc = k == 0 ? xr[0] * m : fmaf(xr[k], m, acc);
            }
            out[r * D + j] = acc;
        }
    }
}

/* Indices go to codes (uint8) or, for codebooks of more than 256 codewords (the reference's int16 /
 * int32 indices, sunshape/codec.py:78-83), to codes32 (one int32 per index). */
static void encode_core(const float* keys, int64_t n, int D, const int64_t* perm, const float* cent,
                        const float* metric, int direct, int nb, int nc, int bd, const uint8_t* heavy, uint8_t* codes,
                        int32_t* codes32, float* pt) {
    float* cn = (float*)malloc(sizeof(float) * (size_t)nb * (size_t)nc);
    float* xp = (float*)malloc(sizeof(float) * (size_t)D);
    float* cm = NULL; /* codebook in the metric space, C_b @ E_b^T */
    float y[64];
    if (metric) {
        cm = (float*)malloc(sizeof(float) * (size_t)nb * (size_t)nc * (size_t)bd);
        for (int b = 0; b < nb; ++b)
            for (int j = 0; j < nc; ++j)
                metric_apply(metric + (int64_t)b * bd * D + (int64_t)b * bd, D, cent + ((int64_t)b * nc + j) * bd, bd,
                             cm + ((int64_t)b * nc + j) * bd);
        cent = cm;
    }
    for (int b = 0; b < nb; ++b)
        for (int j = 0; j < nc; ++j)
            cn[b * nc + j] = sq_norm(cent + ((int64_t)b * nc + j) * bd, bd);
    for (int64_t i = 0; i < n; ++i) {
        const float* k = keys + i * D;
        for (int j = 0; j < D; ++j) xp[j] = k[perm[j]];
        for (int b = 0; b < nb; ++b) {
            const float* xb = xp + b * bd;
            if (heavy && heavy[b]) {
                if (codes32) codes32[i * nb + b] = 0;
                else codes[i * nb + b] = 0;
                if (pt)
                    for (int d = 0; d < bd; ++d) pt[(i * nb + b) * bd + d] = xb[d];
                continue;
            }
            if (pt)
                for (int d = 0; d < bd; ++d) pt[(i * nb + b) * bd + d] = 0.0f;
            const float* cb = cent + (int64_t)b * nc * bd;
            if (metric) {
                metric_apply(metric + (int64_t)b * bd * D + (int64_t)b * bd, D, xb, bd, y);
                xb = y;
            }
            float xn = sq_norm(xb, bd);
            float best = INFINITY;
            int best_j = 0;
            for (int j = 0; j < nc; ++j) {
                float v = direct ? direct_dist2(xb, cb + (int64_t)j * bd, bd)
                                 : mm_dist2(xb, xn, cb + (int64_t)j * bd, cn[b * nc + j], bd);
                float dj = sqrtf(v > 0.0f ? v : 0.0f);
                if (dj < best) { /* strict: the first minimum wins */
                    best = dj;
                    best_j = j;
                }
            }
            if (codes32) codes32[i * nb + b] = best_j;
            else codes[i * nb + b] = (uint8_t)best_j;
        }
    }
    free(xp);
    free(cn);
    free(cm);
}

void oracle_encode_ex(const float* keys, int64_t n, int D, const int64_t* perm, const float* cent,
                      const float* metric, int direct, int nb, int nc, int bd, const uint8_t* heavy, uint8_t* codes,
                      float* pt) {
    encode_core(keys, n, D, perm, cent, metric, direct, nb, nc, bd, heavy, codes, NULL, pt);
}

/* The same with int32 indices (any codebook size). */
void oracle_encode_wide(const float* keys, int64_t n, int D, const int64_t* perm, const float* cent,
                        const float* metric, int direct, int nb, int nc, int bd, const uint8_t* heavy,
                        int32_t* codes, float* pt) {
    encode_core(keys, n, D, perm, cent, metric, direct, nb, nc, bd, heavy, NULL, codes, pt);
}

void oracle_encode_metric(const float* keys, int64_t n, int D, const int64_t* perm, const float* cent,
                          const float* metric, int nb, int nc, int bd, const uint8_t* heavy, uint8_t* codes,
                          float* pt) {
    oracle_encode_ex(keys, n, D, perm, cent, metric, 0, nb, nc, bd, heavy, codes, pt);
}

void oracle_encode(const float* keys, int64_t n, int D, const int64_t* perm, const float* cent,
                   int nb, int nc, int bd, const uint8_t* heavy, uint8_t* codes, float* pt) {
    oracle_encode_ex(keys, n, D, perm, cent, NULL, 0, nb, nc, bd, heavy, codes, pt);
}
