// Nearest-codeword encode (SunShapeBlockCodec.quantize, sunshape/codec.py:362-385).
//
// The reference picks, per block, argmin_c torch.cdist(x_b, C_b) with the first index on
// ties.  torch.cdist takes ATen's mm formulation for these sizes:
//   d2[c] = [-2x, |x|^2, 1] . [c, 1, |c|^2]   (fp32 GEMM, K = bd + 2, k ascending, FMA chain)
//   d[c]  = sqrt(max(d2[c], 0))
// with |v|^2 = left-to-right sum of rounded squares.  Every index this file returns is the
// first argmin of d computed with exactly that arithmetic and a correctly rounded sqrt.
// When both of cdist's inputs have at most 25 rows (a call that quantizes at most 25 keys with at
// most 25 codewords, e.g. 16 at 2 bits/dim and block_dim 2) torch evaluates the distance directly
// instead, d2[c] = sum_k (x_k - c_k)^2 with rounded squares summed in k order; the caller asks for
// that with direct_dist, which the exact scan serves.
//
// Two kernels:
//  * k_encode_scan  -- one thread per (key, block), exact formula for all codewords.
//  * k_encode_mfma  -- v_mfma_f32_16x16x4f32 evaluates the augmented GEMM for 16 keys x
//    256 codewords per wave; every codeword whose MFMA value lies within a proven error
//    bound of the row minimum is re-evaluated with the exact formula on the VALU and the
//    winner is chosen among those (lexicographic (d, index)).  The index is therefore
//    exact whatever the MFMA's internal rounding order.
#include "ssq_encode_math.h"

#include <math.h>
#include <string.h>

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

// sq_norm and metric_row (ssq_encode_math.h) for register arrays of N >= bd entries (unrolled,
// static indexes)
template <int N>
__device__ __forceinline__ float sq_norm_n(const float (&v)[N], int bd) {
    float s = v[0] * v[0];
#pragma unroll
    for (int d = 1; d < N; ++d) {
        const float t = v[d] * v[d];
        if (d < bd) s = s + t;
    }
    return s;
}
template <int N>
__device__ __forceinline__ float metric_row_n(const float* e, const float (&x)[N], int bd) {
    float acc = e[0] * x[0];
#pragma unroll
    for (int j = 1; j < N; ++j)
        if (j < bd) acc = __builtin_fmaf(e[j], x[j], acc);
    return acc;
}

struct EncodeParams {
    ssq_encode_args a;
    int nbc;           // blocks per workgroup chunk
    int fold;          // short sequences: all sequences of a KV head share one key range (SsqKeyMap)
    int passes;        // key passes per workgroup (scan)
};

// ---------------------------------------------------------------------------
// exact scan: thread per (key, block); codebook chunk + norms in LDS
// ---------------------------------------------------------------------------
constexpr int kScanThreads = 256;
constexpr int kScanPasses = 16;  // key passes per workgroup (amortises the codebook staging)

__global__ __launch_bounds__(kScanThreads) void k_encode_scan(const EncodeParams p) {
    extern __shared__ __align__(16) float smem[];
    const ssq_encode_args& a = p.a;
    const SsqKeyMap km(a, p.fold);
    const int kv = km.kv;
    const int blk0 = blockIdx.z * p.nbc;
    const int nbc = min(p.nbc, a.n_blocks - blk0);
    const int bd = a.block_dim, nc = a.n_centroids;
    float* cb = smem;                        // [nbc][nc][bd]
    float* cn = cb + (size_t)nbc * nc * bd;  // [nbc][nc]
    const float* cent = a.cent + (int64_t)kv * a.cent_sh + (int64_t)blk0 * nc * bd;
    const float* met = a.metric ? a.metric + (int64_t)kv * a.metric_sh : nullptr;
    const int D = a.head_dim;
    if (met) {  // codebook in the metric space: c' = E_b c, one codeword per thread
        for (int e = threadIdx.x; e < nbc * nc; e += kScanThreads) {
            const int blk = blk0 + e / nc;
            const float* eb = met + (int64_t)blk * bd * D + blk * bd;
            float c[16];
            for (int d = 0; d < bd; ++d) c[d] = cent[(size_t)e * bd + d];
            for (int k = 0; k < bd; ++k) cb[(size_t)e * bd + k] = metric_row(eb + (int64_t)k * D, c, bd);
        }
    } else {
        for (int e = threadIdx.x; e < nbc * nc * bd; e += kScanThreads) cb[e] = cent[e];
    }
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
    for (int pass = 0; pass < p.passes; ++pass) {
        const int i = (blockIdx.x * p.passes + pass) * keys_per_pass + kk;
        if (i >= km.n_keys) return;
        int b, s;
        km.bs(a, i, b, s);
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
        if (met) {
            const float* eb = met + (int64_t)blk * bd * D + blk * bd;
            float y[16];
            for (int k = 0; k < bd; ++k) y[k] = metric_row(eb + (int64_t)k * D, x, bd);
            for (int k = 0; k < bd; ++k) x[k] = y[k];
        }
        const float xn = sq_norm(x, bd);
        const bool direct = a.direct_dist != 0;
        // pass 1: smallest clamped pre-sqrt value max(e, 0) (first index).  A NaN value (a key
        // with a non-finite element or one whose norm overflows) clamps to 0 as in the
        // reference's sqrt(clamp_min(., 0)) followed by its first argmin of a row holding NaN.
        float emin = INFINITY;
        int jm = 0;
        for (int j = 0; j < nc; ++j) {
            const float e = direct ? direct_dist2(x, cbb + j * bd, bd) : mm_dist2(x, xn, cbb + j * bd, cnb[j], bd);
            const float ec = e > 0.f ? e : 0.f;
            if (ec < emin) { emin = ec; jm = j; }
        }
        // pass 2: the first index whose sqrt equals the minimum's (sqrt merges values at most
        // ~2^-22 apart relatively; indices above jm cannot win).  thr bounds that interval.
        const float fstar = dist_of(emin);
        const float thr = emin > 0.f ? emin * (1.0f + 0x1.0p-20f) : 0.f;
        int best = jm;
        for (int j = 0; j < jm; ++j) {
            const float e = direct ? direct_dist2(x, cbb + j * bd, bd) : mm_dist2(x, xn, cbb + j * bd, cnb[j], bd);
            if (e <= thr && dist_of(e) == fstar) { best = j; break; }
        }
        a.codes[crow + blk] = (uint8_t)best;
    }
}

// ---------------------------------------------------------------------------
// MFMA screen + exact certification
// ---------------------------------------------------------------------------
#ifndef SSQ_ENC_PIPE
#define SSQ_ENC_PIPE 1  // 0: each block's MFMAs and reduction back to back (always so with a metric)
#endif
constexpr int kMfmaWaves = 8;
constexpr int kRounds = 8;        // key groups of 16 per wave per workgroup
constexpr int kMaxLight = 128;
constexpr size_t kMfmaSmemCap = 160 * 1024;  // one workgroup of 8 waves per CU

struct MfmaEncodeParams {
    ssq_encode_args a;
    float e1, e2;             // certification error bound: err = e1*|x|^2 + e2*max(min, 0)
    int ys_stride;            // row stride of the keys' metric images in LDS (block metric only)
    int row_codes;            // 1: one chunk holds every light block and code rows take 16-byte stores
    int nbc;                  // light blocks per workgroup chunk
    int n_light;
    int fold;                 // short sequences: all sequences of a KV head share one key range (SsqKeyMap)
    uint8_t light[kMaxLight]; // light (VQ-coded) block ids, ascending
};

// Exchange with the lane 16 (32) apart through the gfx950 permlane swaps: the two results are this
// lane's value and its partner's, in an order that differs between partners, so only symmetric
// combinations (min, sum, lexicographic min) are taken of them.
__device__ __forceinline__ void xchg16(int v, int& a, int& b) {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    a = (int)r[0];
    b = (int)r[1];
}
__device__ __forceinline__ void xchg32(int v, int& a, int& b) {
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    a = (int)r[0];
    b = (int)r[1];
}
// median of three signed ints (v_med3_i32; no builtin exposes the integer form)
__device__ __forceinline__ int med3_i(int a, int b, int c) {
    int r;
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
// minimum / sum over the 4 lanes l % 16 + 16 g (one key's lanes)
__device__ __forceinline__ int key_min_i(int v) {
    int a, b;
    xchg16(v, a, b); v = min(a, b);
    xchg32(v, a, b); return min(a, b);
}
__device__ __forceinline__ int key_sum_i(int v) {
    int a, b;
    xchg16(v, a, b); v = a + b;
    xchg32(v, a, b); return a + b;
}
// lexicographic (value, index) minimum over the key's 4 lanes
__device__ __forceinline__ void key_lexmin(float& bf, int& bn) {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
        int fa, fb, na, nb2;
        if (st == 0) { xchg16(__float_as_int(bf), fa, fb); xchg16(bn, na, nb2); }
        else { xchg32(__float_as_int(bf), fa, fb); xchg32(bn, na, nb2); }
        const float af = __int_as_float(fa), bfv = __int_as_float(fb);
        const bool take_a = af < bfv || (af == bfv && na < nb2);
        bf = take_a ? af : bfv;
        bn = take_a ? na : nb2;
    }
}

// Distances of one light block for the wave's 16 keys.  Codewords are the MFMA's row operand and
// keys its column operand, so acc[nt][i] = d2[key l%16][codeword 16nt + 4(l/16) + i]: each lane
// holds 64 of its key's 256 distances, and a key's 4 lanes sit 16 apart.
// key element k of light block bl for key row m: the permuted key (xs through poff) or, with a
// block metric, its image E_b x staged in ys
template <bool MET>
__device__ __forceinline__ float key_elem(const float* xs, const float* ys, const int* poff, int XS, int YS, int m,
                                          int bl, int bd, int k) {
    return MET ? ys[m * YS + bl * bd + k] : xs[m * XS + poff[bl * bd + k]];
}

// |x|^2 of key row m's light block bl (of its metric image with a block metric): the squares
// of the block's elements rounded and summed left to right
template <int KS, bool MET>
__device__ __forceinline__ float key_norm(const float* xs, const float* ys, const int* poff, int XS, int YS, int m,
                                          int bl, int bd) {
    constexpr int kCB = 4 * KS - 2;  // >= bd
    float x[kCB];
#pragma unroll
    for (int d = 0; d < kCB; ++d) x[d] = key_elem<MET>(xs, ys, poff, XS, YS, m, bl, bd, min(d, bd - 1));
    return sq_norm_n(x, bd);
}

// column operand of light block bl: [-2x, |x|^2, 1, 0..][k = 4s + l/16] of key l%16
template <int KS, bool MET>
__device__ __forceinline__ void col_operand(const float* xs, const float* ys, float xnv, const int* poff, int bl,
                                            int bd, int XS, int YS, int lane, int lane16, float (&av)[KS]) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const int k = 4 * s + (lane >> 4);
        float v;
        if (k < bd) v = -2.0f * key_elem<MET>(xs, ys, poff, XS, YS, lane16, bl, bd, k);
        else if (k == bd) v = xnv;
        else if (k == bd + 1) v = 1.0f;
        else v = 0.0f;
        av[s] = v;
    }
}

// the block's MFMAs into acc; xnv = |x|^2 of this lane's key block (also needed by the reduction)
template <int KS, bool MET>
__device__ __forceinline__ void issue_block(const float* bsw, const float* xs, const float* ys, const int* poff, int bl,
                                            int bd, int XS, int YS, int lane, int lane16, v4f (&acc)[16], float& xnv) {
    float av[KS];
    xnv = key_norm<KS, MET>(xs, ys, poff, XS, YS, lane16, bl, bd);
    col_operand<KS, MET>(xs, ys, xnv, poff, bl, bd, XS, YS, lane, lane16, av);
    const float* bb = bsw + (size_t)bl * KS * 1024;
#pragma unroll
    for (int nt = 0; nt < 16; ++nt) {
        v4f c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s)
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(bb[(s * 16 + nt) * 64 + lane], av[s], c, 0, 0, 0);
        acc[nt] = c;
    }
}

// first-argmin of sqrt(max(d2,0)) for the 16 keys of the wave in one light block; codes -> cs[key][blk]
//
// Fast path (lane: one key, 64 of its codewords):
//  1. the lane's minimum m1 and second minimum m2 of its MFMA values with a 6-bit slot tag in the
//     low mantissa bits (one min and one med3 per value), compared as signed ints: for values >= 0
//     the float bit pattern orders like a signed int, and every negative value orders below them;
//  2. the key's minimum over its 4 lanes with the 8-bit codeword index in place of the tag, and
//     from it a threshold thr that provably contains the exact reference winner (bound below);
//  3. the key is decided when exactly one of its lanes has m1 <= thr and none has m2 <= thr (both
//     with their 8 low bits cleared, which never raises a value that is >= 0 and keeps a negative
//     one negative).  A decided key has exactly one MFMA value <= thr, and that is the minimum.
// Keys with several candidates re-evaluate just those candidates with the reference's fp32 chain
// and a correctly rounded sqrt, in a compact loop (one candidate per lane per trip).
//
// Error bound.  The K = bd + 2 terms of a distance pass through at most K roundings (product and
// sums, any order, even truncation), so |value_j - |x-c_j|^2| <= g*(|x| + |c_j|)^2 with
// g = 1.001*K*2^-23 (Cauchy-Schwarz), the same for the MFMA and for the reference chain, and
// |c_j| <= |x| + |x-c_j|.  Every codeword that can matter has |x-c_j|^2 <= Y = 1.01*max(mn,0) +
// 64*g*|x|^2 (self-consistent because 12*g << 0.01), so its error is <= err = 8*g*|x|^2 + 2*g*Y
// <= e1*|x|^2 + e2*max(mn,0) with e1 = 1.0234*8g, e2 = 1.0234*2g (+ underflow).  The exact winner
// j* has d(j*) <= d(argmin) and sqrt merges values <= 2^-21 apart, hence value_j*(MFMA) <=
// max(mn,0)*(1 + 2^-21) + 4*err.  mt, the minimum with its 8 low bits cleared, satisfies mt <= mn <
// mt*(1 + 2^-15), so thr = max(mt,0)*(1 + 2^-14) + 5*err(mt) + 2^-100 still exceeds that bound:
// every codeword under thr is a candidate, and so is the key's minimum.
template <int KS, bool MET>
__device__ __forceinline__ void reduce_block(const float* bsw, const float* xs, const float* ys, float xnv,
                                             const int* poff, const int* lightL, int bl, int nb, int bd,
                                             int XS, int YS, int lane16, int mrow, float e1, float e2,
                                             const v4f (&acc)[16], uint8_t* cs) {
    const int grp = mrow >> 2;  // this lane's codeword quarter within each tile of 16
    // 1. lane minimum and second minimum (packed: value bits, slot tag 4nt + i in the low 6 bits)
    int m1 = __float_as_int(acc[0][0]) & -64;
    int m2 = 0x7FFFFFFF;
#pragma unroll
    for (int nt = 0; nt < 16; ++nt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (nt == 0 && i == 0) continue;
            const int v = (__float_as_int(acc[nt][i]) & -64) | (4 * nt + i);
            m2 = med3_i(m1, m2, v);  // m1 <= m2: the second minimum of {m1, m2, v}
            m1 = min(m1, v);
        }
    }
    // 2. key minimum with the codeword index 16nt + 4grp + i in the low 8 bits
    const int t1 = m1;
    const int pk = key_min_i((t1 & -256) | ((t1 & 60) << 2) | (grp << 2) | (t1 & 3));
    const float mp = fmaxf(__int_as_float(pk & -256), 0.f);
    const float thr = mp * (1.0f + 0x1.0p-14f) + 5.0f * (e1 * xnv + e2 * mp) + 0x1.0p-100f;
    // 3. decided keys: one lane's minimum under thr, no lane's second minimum under thr.  A key
    // whose norm is not finite (a non-finite element, or an overflow) has no bound: every codeword
    // is a candidate
    const bool wild = !(thr < INFINITY);
    const int flag = (__int_as_float(t1 & -256) <= thr ? 1 : 0) + (__int_as_float(m2 & -256) <= thr ? 2 : 0);
    const bool undecided = key_sum_i(flag) != 1 || wild;
    int code = pk & 255;
    if (__builtin_amdgcn_ballot_w64(undecided)) {  // rare: several candidates -> exact arithmetic decides
        // This lane's candidates of an undecided key (bit 4nt + i).  While its second minimum is
        // over thr the lane holds at most one value <= thr, and then it is the minimum's slot;
        // only a lane with two candidates scans all 64 values.
        uint64_t cand = 0;
        if (wild) {
            cand = ~0ull;
        } else if (undecided) {
            if (flag & 2) {
#pragma unroll
                for (int nt = 0; nt < 16; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        cand |= acc[nt][i] <= thr ? (1ull << (4 * nt + i)) : 0ull;
            } else if (flag & 1) {
                cand = 1ull << (t1 & 63);
            }
        }
        const float* bb = bsw + (size_t)bl * KS * 1024;
        const int kc = bd + 1;
        const float* cnp = bb + (kc >> 2) * 1024 + (kc & 3) * 16;  // |c|^2 row of the codeword operand
        constexpr int kCB = 4 * KS - 2;  // >= bd
        float xk[kCB];                   // -2x of this lane's key block (loop invariant)
#pragma unroll
        for (int d = 0; d < kCB; ++d)
            xk[d] = -2.0f * key_elem<MET>(xs, ys, poff, XS, YS, lane16, bl, bd, min(d, bd - 1));
        float bf = INFINITY;
        int bn = 4096;
#pragma unroll 1
        while (cand) {
            const int pos = __builtin_ctzll(cand);
            cand &= cand - 1;
            const int r = 4 * grp + (pos & 3);  // codeword 16nt + r
            const int nt = pos >> 2;
            const float* cb = bb + nt * 64 + r;
            float cv[kCB];
#pragma unroll
            for (int d = 0; d < kCB; ++d) cv[d] = cb[(min(d, bd - 1) >> 2) * 1024 + (min(d, bd - 1) & 3) * 16];
            const float cnv = cnp[nt * 64 + r];
            // the reference chain: k ascending FMA over [-2x, |x|^2, 1] . [c, 1, |c|^2]
            float d2 = xk[0] * cv[0];
#pragma unroll
            for (int d = 1; d < kCB; ++d)
                if (d < bd) d2 = __builtin_fmaf(xk[d], cv[d], d2);
            d2 = __builtin_fmaf(xnv, 1.0f, d2);
            d2 = __builtin_fmaf(1.0f, cnv, d2);
            const float f = dist_of(d2);
            const int n = 16 * nt + r;
            if (f < bf || (f == bf && n < bn)) { bf = f; bn = n; }
        }
        key_lexmin(bf, bn);
        if (undecided) code = bn;
    }
    if (mrow == 0) cs[lane16 * nb + lightL[bl]] = (uint8_t)code;
}

inline int mfma_ys_stride(const ssq_encode_args& a, int nbc) { return nbc * a.block_dim + 1; }
inline size_t mfma_enc_smem(const ssq_encode_args& a, int nbc, int KS) {
    size_t words = (size_t)nbc * KS * 1024 + a.head_dim + (size_t)nbc * (a.block_dim + 1) +
                   (size_t)kMfmaWaves * 16 * (a.head_dim + 1);
    if (a.metric)  // E_b blocks of the chunk + the keys' metric images
        words += (size_t)nbc * a.block_dim * a.block_dim + (size_t)kMfmaWaves * 16 * mfma_ys_stride(a, nbc);
    return words * 4 + (size_t)kMfmaWaves * 16 * a.n_blocks + 64;
}

template <int KS, bool MET>
__global__ __launch_bounds__(kMfmaWaves * SSQ_WAVE, 1) void k_encode_mfma(const MfmaEncodeParams p) {
    extern __shared__ __align__(16) float smem[];
    const ssq_encode_args& a = p.a;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar loop control
    const SsqKeyMap km(a, p.fold);
    const int kv = km.kv, n_keys = km.n_keys;
    const int chunk = blockIdx.z;
    const int l0 = chunk * p.nbc;
    const int nbc = min(p.nbc, p.n_light - l0);
    const int bd = a.block_dim, D = a.head_dim, nb = a.n_blocks;
    const int XS = D + 1;
    const uint64_t hm0 = a.heavy_mask[0], hm1 = a.heavy_mask[1];
    const bool do_heavy = chunk == 0 && (hm0 | hm1);
    uint64_t cm0 = 0, cm1 = 0;  // light blocks of this chunk
    for (int bl = 0; bl < nbc; ++bl) {
        const int blk = p.light[l0 + bl];
        if (blk < 64) cm0 |= 1ull << blk; else cm1 |= 1ull << (blk - 64);
    }
    const int lo_blk = nbc > 0 ? p.light[l0] : 0;
    const int hi_blk = nbc > 0 ? p.light[l0 + nbc - 1] : -1;

    // LDS: bsw [nbc][KS][16][64] | perm [D] | poff [nbc*bd] | lightL [nbc] | xs [waves][16][XS] |
    //      (MET: em [nbc][bd][bd] | ys [waves][16][YS]) | codes [waves][16][nb]
    float* bsw = smem;
    int* perm_l = reinterpret_cast<int*>(bsw + (size_t)nbc * KS * 1024);
    int* poff = perm_l + D;         // poff[bl*bd + d] = perm[light[bl]*bd + d]: the block's dims in the key row
    int* lightL = poff + nbc * bd;  // light block ids of this chunk
    float* xs_all = reinterpret_cast<float*>(lightL + nbc);
    float* xs = xs_all + wave * 16 * XS;
    float* tail = xs_all + kMfmaWaves * 16 * XS;
    const int YS = MET ? p.ys_stride : 0;
    float* em = tail;                                  // em[bl][k][j] = E_b[k][j] (MET only)
    float* ys = em + (MET ? nbc * bd * bd : 0) + wave * 16 * YS;
    uint8_t* cs = reinterpret_cast<uint8_t*>(tail + (MET ? nbc * bd * bd + kMfmaWaves * 16 * YS : 0)) + wave * 16 * nb;
    if (p.row_codes) {  // heavy blocks keep code 0 in the whole-row writes
        for (int i = lane; i < 4 * nb; i += 64) reinterpret_cast<uint32_t*>(cs)[i] = 0u;
    }

    const float* cent = a.cent + (int64_t)kv * a.cent_sh;
    const int64_t* perm_g = a.perm + (int64_t)kv * a.perm_sh;
    // key rows: lane (m = l/4, quarter q = l%4) loads elements [q*D/4, (q+1)*D/4) of row m, as
    // D/32 16-byte loads (16-bit keys, D = 64 or 128), prefetched one round ahead
    const int esz = a.k_dtype == SSQ_F32 ? 4 : 2;
    const bool vec = (D == 64 || D == 128) && ((a.k_ss * esz) % 16 == 0) && ((a.k_sh * esz) % 16 == 0) &&
                     ((a.k_sb * esz) % 16 == 0) && ((uintptr_t)a.keys % 16 == 0) && esz == 2;
    const int nq = D / 32;  // 16-byte pieces per lane on the vector path
    const int lm = lane >> 2, lq = lane & 3;
    const int s_wg = blockIdx.x * (kMfmaWaves * kRounds * 16);  // first key index of the workgroup
    constexpr int kPre = 4;
    uint4 pre[kPre];
#pragma unroll
    for (int i = 0; i < kPre; ++i) pre[i] = make_uint4(0, 0, 0, 0);
    auto fetch = [&](int round) {
        const int s = s_wg + (round * kMfmaWaves + wave) * 16 + lm;
        if (vec && s < n_keys) {
            const uint4* src = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.keys) +
                                                              km.krow(a, s) + lq * (D / 4));
#pragma unroll
            for (int i = 0; i < kPre; ++i)
                if (i < nq) pre[i] = src[i];  // wave-uniform
        }
    };
    fetch(0);

    // Prologue loads, all in flight together before any is used: the key rows above, the
    // permutation (up to 4 entries per thread), and the first pass of codeword rows (r0 + u kThr
    // + tid of the chunk; a wave's 64 rows lie in one block, whose id is a wave-uniform kernel
    // argument; rows past the end re-read the last one).
    constexpr int kThr = kMfmaWaves * SSQ_WAVE;
    static_assert(kThr % 256 == 0, "codeword passes of whole blocks");
    const int tid = threadIdx.x;
    constexpr int kPv = 4;
    int pv[kPv];
#pragma unroll
    for (int k = 0; k < kPv; ++k) pv[k] = tid + k * kThr < D ? (int)perm_g[tid + k * kThr] : 0;
    constexpr int kCB = 4 * KS - 2;  // >= bd
    constexpr int kRB = 8;
    const int n_rows = nbc * 256;
    float cv[kRB][kCB];
    auto cb_load = [&](int r0) {
#pragma unroll
        for (int u = 0; u < kRB; ++u) {
            const int rw = r0 + u * kThr + wave * SSQ_WAVE;  // the wave's first row
            const int bl = min(rw >> 8, nbc - 1);
            const int r = min(rw + lane, n_rows - 1);
            const float* c = cent + ((int64_t)p.light[l0 + bl] * 256 + (r & 255)) * bd;
#pragma unroll
            for (int d = 0; d < kCB; ++d) cv[u][d] = c[min(d, bd - 1)];
        }
    };
    if (n_rows > 0) cb_load(0);

#pragma unroll
    for (int k = 0; k < kPv; ++k)
        if (tid + k * kThr < D) perm_l[tid + k * kThr] = pv[k];
    for (int j = tid + kPv * kThr; j < D; j += kThr) perm_l[j] = (int)perm_g[j];  // D > 4 kThr
    for (int bl = tid; bl < nbc; bl += kThr) lightL[bl] = p.light[l0 + bl];
    if (MET) {
        const float* met = a.metric + (int64_t)kv * a.metric_sh;
        for (int j = tid; j < nbc * bd * bd; j += kThr) {
            const int bl = j / (bd * bd), r = j - bl * bd * bd;
            const int k = r / bd, jj = r - k * bd;
            const int blk = p.light[l0 + bl];
            em[j] = met[(int64_t)(blk * bd + k) * D + blk * bd + jj];
        }
        __syncthreads();  // em is read by the codeword transform
    }
    // B operands in lane order: bsw[bl][s][nt][l] = [c, 1, |c|^2, 0..][k = 4s + l/16] of codeword 16nt + l%16
    // (with a block metric, c' = E_b c in place of c).  One codeword row per thread per pass.
    for (int r0 = 0; r0 < n_rows; r0 += kRB * kThr) {
        if (r0 > 0) cb_load(r0);
#pragma unroll
        for (int u = 0; u < kRB; ++u) {
            const int r = r0 + u * kThr + tid;
            if (r >= n_rows) break;
            const int bl = r >> 8, j = r & 255;
            float cp[kCB];
#pragma unroll
            for (int d = 0; d < kCB; ++d) cp[d] = cv[u][d];
            if (MET) {
#pragma unroll
                for (int k = 0; k < kCB; ++k)
                    if (k < bd) cp[k] = metric_row_n(em + (bl * bd + k) * bd, cv[u], bd);
            }
            const float cn = sq_norm_n(cp, bd);
            float* dst = bsw + (size_t)bl * KS * 1024 + (j >> 4) * 64 + (j & 15);
#pragma unroll
            for (int k = 0; k < 4 * KS; ++k)
                dst[(k >> 2) * 1024 + (k & 3) * 16] = k < bd ? cp[k] : k == bd ? 1.0f : k == bd + 1 ? cn : 0.0f;
        }
    }
    __syncthreads();
    // poff[bl bd + d] = perm[light[bl] bd + d], from the staged permutation
    for (int j = tid; j < nbc * bd; j += kThr) {
        const int bl = j / bd, d = j - bl * bd;
        poff[j] = perm_l[lightL[bl] * bd + d];
    }
    __syncthreads();

    const int lane16 = lane & 15;
    const int mrow = 4 * (lane >> 4);

    for (int round = 0; round < kRounds; ++round) {
        const int s0 = s_wg + (round * kMfmaWaves + wave) * 16;
        if (s0 >= n_keys) break;  // wave-uniform
        // output rows of this lane's key (s0 + lane / 4), resolved now: a slot-mapping load then
        // overlaps the round's arithmetic instead of delaying the code writes
        int64_t crow_m, prow_m;
        {
            int b, s;
            km.bs(a, min(s0 + lm, n_keys - 1), b, s);
            out_rows(a, b, kv, s, crow_m, prow_m);
        }
        // stage this round's 16 rows (unpermuted, fp32) into xs
        if (vec) {
            float* dst = xs + lm * XS + lq * (D / 4);
            const bool ok = s0 + lm < n_keys;
#pragma unroll
            for (int i = 0; i < kPre; ++i) {
                if (i >= nq) break;  // wave-uniform
                const uint32_t w[4] = {pre[i].x, pre[i].y, pre[i].z, pre[i].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float lo = a.k_dtype == SSQ_BF16 ? __uint_as_float(w[k] << 16) : ssq_f16_to_f32(w[k] & 0xFFFFu);
                    const float hi =
                        a.k_dtype == SSQ_BF16 ? __uint_as_float(w[k] & 0xFFFF0000u) : ssq_f16_to_f32(w[k] >> 16);
                    dst[8 * i + 2 * k] = ok ? lo : 0.f;
                    dst[8 * i + 2 * k + 1] = ok ? hi : 0.f;
                }
            }
            fetch(round + 1 < kRounds ? round + 1 : round);
        } else {  // element loads, 8 in flight per lane before their LDS stores
            constexpr int kB = 8;
            for (int e0 = lane; e0 < 16 * D; e0 += 64 * kB) {
                float v[kB];
#pragma unroll
                for (int u = 0; u < kB; ++u) {
                    const int e = min(e0 + 64 * u, 16 * D - 1);
                    const int m = e / D, j = e - m * D;
                    const int s = min(s0 + m, n_keys - 1);
                    v[u] = ssq_load_elem(a.keys, a.k_dtype, km.krow(a, s) + j);
                }
#pragma unroll
                for (int u = 0; u < kB; ++u) {
                    const int e = e0 + 64 * u;
                    if (e < 16 * D) {
                        const int m = e / D, j = e - m * D;
                        xs[m * XS + j] = s0 + m < n_keys ? v[u] : 0.f;
                    }
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if constexpr (MET) {  // the key blocks' metric images y = E_b x  (lane: key m = lane & 15, blocks lane/16 + 4k)
            for (int bl = lane >> 4; bl < nbc; bl += 4) {
                float x[16];
                for (int d = 0; d < bd; ++d) x[d] = xs[lane16 * XS + poff[bl * bd + d]];
                for (int k = 0; k < bd; ++k) ys[lane16 * YS + bl * bd + k] = metric_row(em + (bl * bd + k) * bd, x, bd);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }

        if constexpr (SSQ_ENC_PIPE && !MET) {
            // software pipeline: the MFMAs of block bl+1 run while the VALU reduces block bl
            v4f accA[16], accB[16];
            float xnA = 0.f, xnB = 0.f;
            if (nbc > 0) issue_block<KS, MET>(bsw, xs, ys, poff, 0, bd, XS, YS, lane, lane16, accA, xnA);
            for (int bl = 0; bl < nbc; bl += 2) {
                if (bl + 1 < nbc) issue_block<KS, MET>(bsw, xs, ys, poff, bl + 1, bd, XS, YS, lane, lane16, accB, xnB);
                reduce_block<KS, MET>(bsw, xs, ys, xnA, poff, lightL, bl, nb, bd, XS, YS, lane16, mrow, p.e1, p.e2, accA, cs);
                if (bl + 1 >= nbc) break;
                if (bl + 2 < nbc) issue_block<KS, MET>(bsw, xs, ys, poff, bl + 2, bd, XS, YS, lane, lane16, accA, xnA);
                reduce_block<KS, MET>(bsw, xs, ys, xnB, poff, lightL, bl + 1, nb, bd, XS, YS, lane16, mrow, p.e1, p.e2, accB, cs);
            }
        } else {
            for (int bl = 0; bl < nbc; ++bl) {
                v4f acc[16];
                float xnv;
                issue_block<KS, MET>(bsw, xs, ys, poff, bl, bd, XS, YS, lane, lane16, acc, xnv);
                reduce_block<KS, MET>(bsw, xs, ys, xnv, poff, lightL, bl, nb, bd, XS, YS, lane16, mrow, p.e1, p.e2, acc, cs);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // write this round's codes.  Whole rows: the wave's code rows, complete in cs (heavy
        // entries hold 0), go out in 16-byte pieces, then the passthrough values.  Otherwise lane
        // (key m = lane/4) writes blocks lane%4 + 4k of its key, and chunk 0 also writes the heavy
        // blocks' code 0 and passthrough values.
        if (p.row_codes) {
            const int pieces = nb >> 4;
            for (int e0 = 0; e0 < 16 * pieces; e0 += 64) {  // every lane runs every trip (the shuffles)
                const int e = min(e0 + lane, 16 * pieces - 1);
                const int m = e / pieces, q = e - m * pieces;
                const int i = s0 + m;
                const uint32_t clo = (uint32_t)__shfl((int)(uint32_t)crow_m, 4 * m);  // key m's row, from lane 4m
                const uint32_t chi = (uint32_t)__shfl((int)(uint32_t)((uint64_t)crow_m >> 32), 4 * m);
                const int64_t crow = (int64_t)(((uint64_t)chi << 32) | clo);
                if (e0 + lane < 16 * pieces && i < n_keys) {
                    const uint32_t* src = reinterpret_cast<const uint32_t*>(cs + m * nb + 16 * q);
                    *reinterpret_cast<uint4*>(a.codes + crow + 16 * q) = make_uint4(src[0], src[1], src[2], src[3]);
                }
            }
            const int m = lane >> 2;
            const int i = s0 + m;
            if (do_heavy && i < n_keys) {
                const int64_t prow = prow_m;
                for (int blk = lane & 3; blk < nb; blk += 4) {
                    if (!ssq_is_heavy(hm0, hm1, blk)) continue;
                    const int slot = a.pt_dense ? blk : heavy_ordinal(hm0, hm1, blk);
                    for (int d = 0; d < bd; ++d)
                        ssq_store_elem(a.pt, a.pt_dtype, prow + (int64_t)slot * bd + d, xs[m * XS + perm_l[blk * bd + d]]);
                }
            }
        } else {
            const int m = lane >> 2;
            const int i = s0 + m;
            if (i < n_keys) {
                const int64_t crow = crow_m, prow = prow_m;
                for (int blk = lane & 3; blk < nb; blk += 4) {
                    const bool heavy = ssq_is_heavy(hm0, hm1, blk);
                    if (heavy) {
                        if (!do_heavy) continue;
                        a.codes[crow + blk] = 0;
                        const int slot = a.pt_dense ? blk : heavy_ordinal(hm0, hm1, blk);
                        for (int d = 0; d < bd; ++d)
                            ssq_store_elem(a.pt, a.pt_dtype, prow + (int64_t)slot * bd + d, xs[m * XS + perm_l[blk * bd + d]]);
                    } else if (blk >= lo_blk && blk <= hi_blk && ((blk < 64 ? (cm0 >> blk) : (cm1 >> (blk - 64))) & 1ull)) {
                        a.codes[crow + blk] = cs[m * nb + blk];
                    }
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

constexpr size_t kMaxSmem = 160 * 1024;


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
    SSQ_REQUIRE(a->n_centroids >= 1 && a->n_centroids <= kMaxCentroids, "n_centroids must be in [1, %d]", kMaxCentroids);
    const bool any_heavy = a->heavy_mask[0] || a->heavy_mask[1];
    SSQ_REQUIRE(!any_heavy || a->pt, "heavy blocks need a passthrough output");
    if (any_heavy) SSQ_REQUIRE(a->pt_dtype >= SSQ_F32 && a->pt_dtype <= SSQ_F16, "bad pt_dtype");
    if (a->slot_mapping) SSQ_REQUIRE(a->page_size >= 1, "paged output needs page_size >= 1");
    SSQ_REQUIRE(a->direct_dist == 0 || a->direct_dist == 1, "direct_dist must be 0 or 1");
    if (a->batch == 0 || a->seq_len == 0) return SSQ_OK;
    hipStream_t st = (hipStream_t)stream;
    // the direct distance (a cdist over at most 25 x 25 rows) runs on the exact scan only: the MFMA
    // screen and the grid search certify candidates against the mm formulation's rounding
    SSQ_UNSUPPORTED(!a->direct_dist || a->kernel == 0 || a->kernel == 1,
                    "direct_dist runs on the exact scan (kernel 0 or 1), not kernel %d", a->kernel);
    if (a->n_centroids > 256) {  // 16- / 32-bit codes: the chunked exact scan
        SSQ_UNSUPPORTED(a->kernel == 0 || a->kernel == 1,
                        "n_centroids=%d encodes on the exact scan (kernel 0 or 1), not kernel %d", a->n_centroids,
                        a->kernel);
        const int cw = ssq_code_width(a->n_centroids);
        SSQ_REQUIRE((uintptr_t)a->codes % cw == 0, "%d-bit codes must be %d-byte aligned", 8 * cw, cw);
        return ssq_encode_wide_run(a, st);
    }
    if (!a->direct_dist && (a->kernel == 3 || (a->kernel == 0 && a->grid && ssq_encode_grid_supported(a))))
        return ssq_encode_grid_run(a, st);
    EncodeParams p;
    p.a = *a;
    const int KS = (a->block_dim + 2 + 3) / 4;
    const bool mfma_ok = a->n_centroids == 256 && KS <= 3 && !a->direct_dist;
    const int kernel = a->kernel == 0 ? (mfma_ok ? 2 : 1) : a->kernel;
    if (kernel == 2) {
        SSQ_UNSUPPORTED(mfma_ok, "MFMA encode needs n_centroids == 256 and block_dim <= 10");
        MfmaEncodeParams mp;
        memset(&mp, 0, sizeof(mp));
        mp.a = *a;
        {
            // g = 1.001 * K * 2^-23 for the K = bd + 2 terms of a distance; 1.0234 covers the
            // bound's second-order terms (see reduce_block); rounded up by the 1.0005 factor
            const double g = 1.001 * (a->block_dim + 2) * 0x1.0p-23;
            mp.e1 = (float)(1.0234 * 8.0 * g * 1.0005);
            mp.e2 = (float)(1.0234 * 2.0 * g * 1.0005);
        }
        mp.n_light = 0;
        for (int blk = 0; blk < a->n_blocks; ++blk) {
            const bool heavy = blk < 64 ? ((a->heavy_mask[0] >> blk) & 1) : ((a->heavy_mask[1] >> (blk - 64)) & 1);
            if (!heavy) mp.light[mp.n_light++] = (uint8_t)blk;
        }
        int nbc = mp.n_light > 0 ? mp.n_light : 1;
        while (nbc > 1 && mfma_enc_smem(*a, nbc, KS) > kMfmaSmemCap) --nbc;
        if (mp.n_light > 0) {  // balance the chunks
            const int chunks0 = (mp.n_light + nbc - 1) / nbc;
            nbc = (mp.n_light + chunks0 - 1) / chunks0;
        }
        SSQ_UNSUPPORTED(mfma_enc_smem(*a, nbc, KS) <= kMaxSmem, "head_dim too large for the MFMA encode");
        const int keys_wg = kMfmaWaves * kRounds * 16;
        mp.fold = ssq_encode_fold(a, keys_wg);
        const int64_t n_keys = mp.fold ? (int64_t)a->batch * a->seq_len : a->seq_len;
        const int64_t groups = ((n_keys + keys_wg - 1) / keys_wg) * (mp.fold ? a->num_kv_heads : a->batch * a->num_kv_heads);
        if (mp.n_light > 0 && groups * ((mp.n_light + nbc - 1) / nbc) < ssq_device_cus()) {
            // a small launch (a decode step's append): more, smaller block chunks fill the chip
            const int64_t want = (ssq_device_cus() + groups - 1) / groups;
            const int chunks1 = (int)(want < mp.n_light ? want : mp.n_light);
            nbc = (mp.n_light + chunks1 - 1) / chunks1;
        }
        mp.nbc = nbc;
        mp.ys_stride = mfma_ys_stride(*a, nbc);
        const int chunks = mp.n_light > 0 ? (mp.n_light + nbc - 1) / nbc : 1;
        mp.row_codes = chunks == 1 && a->n_blocks % 16 == 0 && (uintptr_t)a->codes % 16 == 0 && a->c_sb % 16 == 0 &&
                       a->c_sh % 16 == 0 && a->c_st % 16 == 0;
        dim3 grid((unsigned)((n_keys + keys_wg - 1) / keys_wg), mp.fold ? a->num_kv_heads : a->batch * a->num_kv_heads,
                  chunks);
        const size_t smem = mfma_enc_smem(*a, nbc, KS);
        int rc;
        const int sel = KS * 2 + (a->metric ? 1 : 0);
        switch (sel) {
#define SSQ_ENC_LAUNCH(KSV, MV)                                                                        \
    case KSV * 2 + MV: {                                                                               \
        rc = ssq_allow_lds((const void*)k_encode_mfma<KSV, MV>, (int)kMaxSmem, "hipFuncSetAttribute(encode)"); \
        if (rc) return rc;                                                                             \
        hipLaunchKernelGGL((k_encode_mfma<KSV, MV>), grid, dim3(kMfmaWaves * SSQ_WAVE), smem, st, mp); \
        break;                                                                                         \
    }
            SSQ_ENC_LAUNCH(1, false)
            SSQ_ENC_LAUNCH(1, true)
            SSQ_ENC_LAUNCH(2, false)
            SSQ_ENC_LAUNCH(2, true)
            SSQ_ENC_LAUNCH(3, false)
            SSQ_ENC_LAUNCH(3, true)
#undef SSQ_ENC_LAUNCH
            default: return ssq_fail(SSQ_ERR_UNSUPPORTED, "MFMA encode: unsupported block_dim");
        }
        return ssq_check_hip(hipGetLastError(), "k_encode_mfma launch");
    }
    // exact scan
    int nbc = a->n_blocks < kScanThreads ? a->n_blocks : kScanThreads;
    while (nbc > 1 && (size_t)nbc * a->n_centroids * (a->block_dim + 1) * 4 > 96 * 1024) --nbc;
    p.nbc = nbc;
    // folded (short sequences): one pass per workgroup, so the few keys spread over workgroups
    p.fold = ssq_encode_fold(a, (kScanThreads / nbc) * kScanPasses);
    p.passes = p.fold ? 1 : kScanPasses;
    const int keys_per_wg = (kScanThreads / nbc) * p.passes;
    const int64_t n_keys = p.fold ? (int64_t)a->batch * a->seq_len : a->seq_len;
    dim3 grid((unsigned)((n_keys + keys_per_wg - 1) / keys_per_wg), p.fold ? a->num_kv_heads : a->batch * a->num_kv_heads,
              (a->n_blocks + nbc - 1) / nbc);
    const size_t smem = (size_t)nbc * a->n_centroids * (a->block_dim + 1) * 4;
    int rc = ssq_allow_lds((const void*)k_encode_scan, (int)kMaxSmem, "hipFuncSetAttribute(encode)");
    if (rc) return rc;
    hipLaunchKernelGGL(k_encode_scan, grid, dim3(kScanThreads), smem, st, p);
    return ssq_check_hip(hipGetLastError(), "k_encode_scan launch");
}
