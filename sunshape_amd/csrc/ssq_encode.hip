// Nearest-codeword encode (SunShapeBlockCodec.quantize, sunshape/codec.py:362-385).
//
// The reference picks, per block, argmin_c torch.cdist(x_b, C_b) with the first index on
// ties.  torch.cdist takes ATen's mm formulation for these sizes:
//   d2[c] = [-2x, |x|^2, 1] . [c, 1, |c|^2]   (fp32 GEMM, K = bd + 2, k ascending, FMA chain)
//   d[c]  = sqrt(max(d2[c], 0))
// with |v|^2 = left-to-right sum of rounded squares.  Every index this file returns is the
// first argmin of d computed with exactly that arithmetic and a correctly rounded sqrt.
//
// Two kernels:
//  * k_encode_scan  -- one thread per (key, block), exact formula for all codewords.
//  * k_encode_mfma  -- v_mfma_f32_16x16x4f32 evaluates the augmented GEMM for 16 keys x
//    256 codewords per wave; every codeword whose MFMA value lies within a proven error
//    bound of the row minimum is re-evaluated with the exact formula on the VALU and the
//    winner is chosen among those (lexicographic (d, index)).  The index is therefore
//    exact whatever the MFMA's internal rounding order.
#include "ssq_common.h"

#include <math.h>

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

// |v|^2 as x.pow(2).sum(-1): squares rounded, summed left to right (no contraction:
// this file is compiled with -ffp-contract=off)
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

// correctly rounded sqrt of max(v, 0)
__device__ __forceinline__ float dist_of(float v) { return __builtin_sqrtf(v > 0.f ? v : 0.f); }

struct EncodeParams {
    ssq_encode_args a;
    int nbc;           // blocks per workgroup chunk
};

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

// ---------------------------------------------------------------------------
// exact scan: thread per (key, block); codebook chunk + norms in LDS
// ---------------------------------------------------------------------------
constexpr int kScanThreads = 256;
constexpr int kScanPasses = 16;  // key passes per workgroup (amortises the codebook staging)

__global__ __launch_bounds__(kScanThreads) void k_encode_scan(const EncodeParams p) {
    extern __shared__ __align__(16) float smem[];
    const ssq_encode_args& a = p.a;
    const int bk = blockIdx.y;
    const int b = bk / a.num_kv_heads, kv = bk - b * a.num_kv_heads;
    const int blk0 = blockIdx.z * p.nbc;
    const int nbc = min(p.nbc, a.n_blocks - blk0);
    const int bd = a.block_dim, nc = a.n_centroids;
    float* cb = smem;                        // [nbc][nc][bd]
    float* cn = cb + (size_t)nbc * nc * bd;  // [nbc][nc]
    const float* cent = a.cent + (int64_t)kv * a.cent_sh + (int64_t)blk0 * nc * bd;
    for (int e = threadIdx.x; e < nbc * nc * bd; e += kScanThreads) cb[e] = cent[e];
    __syncthreads();
    for (int e = threadIdx.x; e < nbc * nc; e += kScanThreads) cn[e] = sq_norm(cb + (size_t)e * bd, bd);
    __syncthreads();

    const int64_t* perm = a.perm + (int64_t)kv * a.perm_sh;
    const int keys_per_pass = kScanThreads / nbc;
    const int kk = threadIdx.x / nbc, bl = threadIdx.x - kk * nbc;
    if (kk >= keys_per_pass) return;
    const int blk = blk0 + bl;
    const bool heavy = ssq_is_heavy(a.heavy_mask[0], a.heavy_mask[1], blk);
    const float* cbb = cb + (size_t)bl * nc * bd;
    const float* cnb = cn + (size_t)bl * nc;
    for (int pass = 0; pass < kScanPasses; ++pass) {
        const int s = (blockIdx.x * kScanPasses + pass) * keys_per_pass + kk;
        if (s >= a.seq_len) return;
        const int64_t kbase = (int64_t)b * a.k_sb + (int64_t)kv * a.k_sh + (int64_t)s * a.k_ss;
        float x[16];
        for (int d = 0; d < bd; ++d) x[d] = ssq_load_elem(a.keys, a.k_dtype, kbase + perm[blk * bd + d]);
        int64_t crow, prow;
        out_rows(a, b, kv, s, crow, prow);
        if (heavy) {
            a.codes[crow + blk] = 0;
            const int slot = a.pt_dense ? blk : heavy_ordinal(a.heavy_mask[0], a.heavy_mask[1], blk);
            for (int d = 0; d < bd; ++d) ssq_store_elem(a.pt, a.pt_dtype, prow + (int64_t)slot * bd + d, x[d]);
            continue;
        }
        const float xn = sq_norm(x, bd);
        // pass 1: smallest pre-sqrt value (first index)
        float emin = INFINITY;
        int jm = 0;
        for (int j = 0; j < nc; ++j) {
            const float e = mm_dist2(x, xn, cbb + j * bd, cnb[j], bd);
            if (e < emin) { emin = e; jm = j; }
        }
        // pass 2: the first index whose sqrt equals the minimum's (sqrt merges values at most
        // ~2^-22 apart relatively; indices above jm cannot win).  thr bounds that interval.
        const float fstar = dist_of(emin);
        const float thr = emin > 0.f ? emin * (1.0f + 0x1.0p-20f) : 0.f;
        int best = jm;
        for (int j = 0; j < jm; ++j) {
            const float e = mm_dist2(x, xn, cbb + j * bd, cnb[j], bd);
            if (e <= thr && dist_of(e) == fstar) { best = j; break; }
        }
        a.codes[crow + blk] = (uint8_t)best;
    }
}

// ---------------------------------------------------------------------------
// MFMA screen + exact certification
// ---------------------------------------------------------------------------
constexpr int kMfmaWaves = 4;
constexpr int kRounds = 8;  // key groups of 16 per wave per workgroup

template <int KS>
__global__ __launch_bounds__(kMfmaWaves * SSQ_WAVE) void k_encode_mfma(const EncodeParams p) {
    extern __shared__ __align__(16) float smem[];
    const ssq_encode_args& a = p.a;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int bk = blockIdx.y;
    const int b = bk / a.num_kv_heads, kv = bk - b * a.num_kv_heads;
    const int blk0 = blockIdx.z * p.nbc;
    const int nbc = min(p.nbc, a.n_blocks - blk0);
    const int bd = a.block_dim, D = a.head_dim, nb = a.n_blocks;
    const int XS = D + 1;  // padded row stride of the per-wave key scratch
    const uint64_t hm0 = a.heavy_mask[0], hm1 = a.heavy_mask[1];

    // LDS: bsw [nbc][KS][16][64] | cnmax [nbc] | xs [waves][16][XS] | xn [waves][16][nb] | codes [waves][16][nbc]
    float* bsw = smem;
    float* cnmax = bsw + (size_t)nbc * KS * 16 * 64;
    float* xs_all = cnmax + nbc;
    float* xn_all = xs_all + kMfmaWaves * 16 * XS;
    uint8_t* codes_all = reinterpret_cast<uint8_t*>(xn_all + kMfmaWaves * 16 * nb);

    // B operands in lane order: bsw[bl][s][nt][l] = Baug[k = 4s + l/16][n = 16nt + l%16]
    const float* cent = a.cent + (int64_t)kv * a.cent_sh;
    for (int e = threadIdx.x; e < nbc * KS * 16 * 64; e += kMfmaWaves * SSQ_WAVE) {
        const int l = e & 63;
        const int nt = (e >> 6) & 15;
        const int s = (e >> 10) % KS;
        const int bl = e / (KS * 1024);
        const int blk = blk0 + bl;
        const int k = 4 * s + (l >> 4);
        const int n = 16 * nt + (l & 15);
        const float* c = cent + ((int64_t)blk * 256 + n) * bd;
        float v;
        if (k < bd) v = c[k];
        else if (k == bd) v = 1.0f;
        else if (k == bd + 1) v = sq_norm(c, bd);
        else v = 0.0f;
        bsw[e] = v;
    }
    __syncthreads();
    for (int bl = threadIdx.x; bl < nbc; bl += kMfmaWaves * SSQ_WAVE) {
        float m = 0.f;
        const float* c = cent + (int64_t)(blk0 + bl) * 256 * bd;
        for (int n = 0; n < 256; ++n) m = fmaxf(m, sq_norm(c + n * bd, bd));
        cnmax[bl] = m;
    }

    float* xs = xs_all + wave * 16 * XS;
    float* xn = xn_all + wave * 16 * nb;
    uint8_t* cs = codes_all + wave * 16 * nbc;
    const int64_t* perm = a.perm + (int64_t)kv * a.perm_sh;
    const int s_wg = blockIdx.x * (kMfmaWaves * kRounds * 16);

    for (int round = 0; round < kRounds; ++round) {
        const int s0 = s_wg + (round * kMfmaWaves + wave) * 16;
        // stage 16 keys (permuted, fp32) and their block norms
        for (int e = lane; e < 16 * D; e += 64) {
            const int m = e / D, j = e - m * D;
            const int s = s0 + m;
            float v = 0.f;
            if (s < a.seq_len)
                v = ssq_load_elem(a.keys, a.k_dtype,
                                  (int64_t)b * a.k_sb + (int64_t)kv * a.k_sh + (int64_t)s * a.k_ss + perm[j]);
            xs[m * XS + j] = v;
        }
        __syncthreads();
        for (int e = lane; e < 16 * nb; e += 64) {
            const int m = e / nb, blk = e - m * nb;
            xn[e] = sq_norm(xs + m * XS + blk * bd, bd);
        }
        __syncthreads();

        for (int bl = 0; bl < nbc; ++bl) {
            const int blk = blk0 + bl;
            if (ssq_is_heavy(hm0, hm1, blk)) {
                if (lane < 16) cs[lane * nbc + bl] = 0;
                continue;
            }
            // A operand: lane (m = l%16, k = 4s + l/16) holds [-2x, xn, 1, 0...][k]
            const int am = lane & 15;
            float av[KS];
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const int k = 4 * s + (lane >> 4);
                float v;
                if (k < bd) v = -2.0f * xs[am * XS + blk * bd + k];
                else if (k == bd) v = xn[am * nb + blk];
                else if (k == bd + 1) v = 1.0f;
                else v = 0.0f;
                av[s] = v;
            }
            const float* bb = bsw + (size_t)bl * KS * 1024;
            v4f acc[16];
#pragma unroll
            for (int nt = 0; nt < 16; ++nt) {
                v4f c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < KS; ++s)
                    c = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s], bb[(s * 16 + nt) * 64 + lane], c, 0, 0, 0);
                acc[nt] = c;
            }
            // lane holds d2[m = 4*(l/16) + i][n = 16*nt + l%16]
            float mn[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v = acc[0][i];
#pragma unroll
                for (int nt = 1; nt < 16; ++nt) v = fminf(v, acc[nt][i]);
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) v = fminf(v, __shfl_xor(v, o, 64));
                mn[i] = v;
            }
            // Any fp32 evaluation of the K <= 12 term sum (by the MFMA or the exact chain)
            // is within 12*2u*(sum |terms|) <= 50u*(xn + cn) of the real value; eps uses 256u.
            // The exact winner's MFMA value is <= min + 3 eps + 2^-21 (min + eps).
            float thr[4];
            const int mrow = 4 * (lane >> 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float eps = 0x1.0p-16f * (xn[(mrow + i) * nb + blk] + cnmax[bl]) + 0x1.0p-100f;
                thr[i] = mn[i] + 4.0f * eps + 0x1.0p-20f * fabsf(mn[i]);
            }
            float bf[4];
            int bn[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) { bf[i] = INFINITY; bn[i] = 256; }
#pragma unroll
            for (int nt = 0; nt < 16; ++nt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (acc[nt][i] <= thr[i]) {
                        const int m = mrow + i;
                        const int n = 16 * nt + (lane & 15);
                        float x[12], c[12];
                        for (int d = 0; d < bd; ++d) {
                            x[d] = xs[m * XS + blk * bd + d];
                            const int k = d;
                            c[d] = bb[((k >> 2) * 16 + nt) * 64 + (k & 3) * 16 + (lane & 15)];
                        }
                        const int kc = bd + 1;
                        const float cnv = bb[((kc >> 2) * 16 + nt) * 64 + (kc & 3) * 16 + (lane & 15)];
                        const float f = dist_of(mm_dist2(x, xn[m * nb + blk], c, cnv, bd));
                        if (f < bf[i] || (f == bf[i] && n < bn[i])) { bf[i] = f; bn[i] = n; }
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) {
                    const float of = __shfl_xor(bf[i], o, 64);
                    const int on = __shfl_xor(bn[i], o, 64);
                    if (of < bf[i] || (of == bf[i] && on < bn[i])) { bf[i] = of; bn[i] = on; }
                }
            }
            if ((lane & 15) == 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i) cs[(mrow + i) * nbc + bl] = (uint8_t)bn[i];
            }
        }
        __syncthreads();
        // write codes (and passthrough values) for the 16 keys of this round
        for (int e = lane; e < 16 * nbc; e += 64) {
            const int m = e / nbc, bl = e - m * nbc;
            const int s = s0 + m;
            if (s >= a.seq_len) continue;
            const int blk = blk0 + bl;
            int64_t crow, prow;
            out_rows(a, b, kv, s, crow, prow);
            a.codes[crow + blk] = cs[e];
            if (ssq_is_heavy(hm0, hm1, blk)) {
                const int slot = a.pt_dense ? blk : heavy_ordinal(hm0, hm1, blk);
                for (int d = 0; d < bd; ++d)
                    ssq_store_elem(a.pt, a.pt_dtype, prow + (int64_t)slot * bd + d, xs[m * XS + blk * bd + d]);
            }
        }
        __syncthreads();
    }
}

constexpr size_t kMaxSmem = 160 * 1024;

size_t mfma_smem(const ssq_encode_args& a, int nbc, int KS) {
    return ((size_t)nbc * KS * 1024 + nbc + (size_t)kMfmaWaves * 16 * (a.head_dim + 1) +
            (size_t)kMfmaWaves * 16 * a.n_blocks) * 4 + (size_t)kMfmaWaves * 16 * nbc + 16;
}

template <typename K>
int set_smem_attr(K kern, bool& done) {
    if (done) return SSQ_OK;
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxSmem);
    if (e != hipSuccess) return ssq_check_hip(e, "hipFuncSetAttribute(encode)");
    done = true;
    return SSQ_OK;
}

}  // namespace

extern "C" int ssq_encode(const ssq_encode_args* a, void* stream) {
    if (!a) return ssq_fail(SSQ_ERR_INVALID, "args is NULL");
    if (a->struct_size != sizeof(ssq_encode_args))
        return ssq_fail(SSQ_ERR_ABI, "ssq_encode_args size %u != library's %zu", a->struct_size, sizeof(ssq_encode_args));
    SSQ_REQUIRE(a->keys && a->perm && a->cent && a->codes, "keys, perm, cent and codes must be non-NULL");
    SSQ_REQUIRE(a->batch >= 0 && a->num_kv_heads >= 1 && a->seq_len >= 0, "bad batch/heads/seq_len");
    SSQ_REQUIRE(a->k_dtype >= SSQ_F32 && a->k_dtype <= SSQ_F16, "bad k_dtype");
    SSQ_REQUIRE(a->block_dim >= 1 && a->block_dim <= 16 && a->head_dim % a->block_dim == 0,
                "head_dim must be divisible by block_dim (block_dim <= 16)");
    SSQ_REQUIRE(a->n_blocks == a->head_dim / a->block_dim && a->n_blocks <= 128, "bad n_blocks");
    SSQ_REQUIRE(a->n_centroids >= 1 && a->n_centroids <= 256, "n_centroids must be in [1, 256] for uint8 codes");
    const bool any_heavy = a->heavy_mask[0] || a->heavy_mask[1];
    SSQ_REQUIRE(!any_heavy || a->pt, "heavy blocks need a passthrough output");
    if (any_heavy) SSQ_REQUIRE(a->pt_dtype >= SSQ_F32 && a->pt_dtype <= SSQ_F16, "bad pt_dtype");
    if (a->slot_mapping) SSQ_REQUIRE(a->page_size >= 1, "paged output needs page_size >= 1");
    if (a->batch == 0 || a->seq_len == 0) return SSQ_OK;
    hipStream_t st = (hipStream_t)stream;
    EncodeParams p;
    p.a = *a;
    const int KS = (a->block_dim + 2 + 3) / 4;
    const bool mfma_ok = a->n_centroids == 256 && KS <= 3;
    const int kernel = a->kernel == 0 ? (mfma_ok ? 2 : 1) : a->kernel;
    if (kernel == 2) {
        SSQ_UNSUPPORTED(mfma_ok, "MFMA encode needs n_centroids == 256 and block_dim <= 10");
        int nbc = a->n_blocks;
        while (nbc > 1 && mfma_smem(*a, nbc, KS) > kMaxSmem) --nbc;
        SSQ_UNSUPPORTED(mfma_smem(*a, nbc, KS) <= kMaxSmem, "head_dim too large for the MFMA encode");
        p.nbc = nbc;
        const int keys_wg = kMfmaWaves * kRounds * 16;
        dim3 grid((a->seq_len + keys_wg - 1) / keys_wg, a->batch * a->num_kv_heads, (a->n_blocks + nbc - 1) / nbc);
        const size_t smem = mfma_smem(*a, nbc, KS);
        int rc;
        switch (KS) {
            case 1: { static bool d = false; rc = set_smem_attr(k_encode_mfma<1>, d); if (rc) return rc;
                      hipLaunchKernelGGL(k_encode_mfma<1>, grid, dim3(kMfmaWaves * SSQ_WAVE), smem, st, p); break; }
            case 2: { static bool d = false; rc = set_smem_attr(k_encode_mfma<2>, d); if (rc) return rc;
                      hipLaunchKernelGGL(k_encode_mfma<2>, grid, dim3(kMfmaWaves * SSQ_WAVE), smem, st, p); break; }
            default: { static bool d = false; rc = set_smem_attr(k_encode_mfma<3>, d); if (rc) return rc;
                       hipLaunchKernelGGL(k_encode_mfma<3>, grid, dim3(kMfmaWaves * SSQ_WAVE), smem, st, p); break; }
        }
        return ssq_check_hip(hipGetLastError(), "k_encode_mfma launch");
    }
    // exact scan
    int nbc = a->n_blocks < kScanThreads ? a->n_blocks : kScanThreads;
    while (nbc > 1 && (size_t)nbc * a->n_centroids * (a->block_dim + 1) * 4 > 96 * 1024) --nbc;
    p.nbc = nbc;
    const int keys_per_wg = (kScanThreads / nbc) * kScanPasses;
    dim3 grid((a->seq_len + keys_per_wg - 1) / keys_per_wg, a->batch * a->num_kv_heads,
              (a->n_blocks + nbc - 1) / nbc);
    const size_t smem = (size_t)nbc * a->n_centroids * (a->block_dim + 1) * 4;
    static bool done = false;
    int rc = set_smem_attr(k_encode_scan, done);
    if (rc) return rc;
    hipLaunchKernelGGL(k_encode_scan, grid, dim3(kScanThreads), smem, st, p);
    return ssq_check_hip(hipGetLastError(), "k_encode_scan launch");
}
