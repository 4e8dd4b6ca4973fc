// VQ-key decode attention: LUT build in LDS + code gather-sum + online softmax + P.V.
//
// Generic kernel (any head grouping, block_dim, contiguous or paged layout).
// One workgroup = (split of the context) x (group of <= 8 query rows) x (batch, KV head).
//   1. q rows -> scaled/rounded like the reference (vllm_attn_backend.py:235-236),
//      permuted into the codec basis (codec.py:247-252), kept in LDS.
//   2. LUT[blk][c][r] = q_perm[r, blk] . C[blk, c]   (triton_kernels.py:381-408), in LDS.
//   3. For each 256-token tile (one token per thread): score = sum_blk LUT[blk][code]
//      in block order (triton_kernels.py:174-196), + passthrough blocks, + mask;
//      optional raw-score store; online softmax; P.V accumulated in fp32.
//   4. Per split: normalised output + lse, or (m, l, o) partials merged by k_merge.
// Codebooks of more than 256 codewords (16- or 32-bit codes, ssq_code_width) have no LUT: a
// nb x nc x RP table would not fit the LDS (4,096 codewords at 32 blocks: 512 KiB per query row).
// Each token's codewords are gathered from the codebook in global memory instead (L2 / Infinity
// Cache resident: 2 MiB per head at 4,096 codewords of dim 4 and 32 blocks) and dotted with the
// query rows block by block: the LUT entry's FMA chain from the first product, summed in block
// order, so the scores are the LUT path's arithmetic.
#include "ssq_common.h"

#include <math.h>

namespace {

constexpr int kThreads = 256;
constexpr int kTile = 256;   // tokens per main-loop iteration
constexpr int kMaxRows = 8;  // query rows per workgroup (LUT is [nb][nc][RP])

struct DecodeParams {
    ssq_decode_args a;
    int G;          // query heads per KV head
    int rows;       // G * q_len rows per (batch, KV head)
    int R;          // rows per workgroup
    int split_len;  // tokens per split (multiple of kTile)
    int n_splits;
    int word_codes; // 1: code rows are 4-byte aligned with nb % 4 == 0
    int vec_cent;   // 1: codebook 16-byte aligned (per head too), head_dim % 4 == 0, nb*nc % 4 == 0
    int cw;         // code width in bytes (ssq_code_width): > 1 gathers codewords instead of a LUT
    float* ws_o;    // [n_splits, B*Hq*Lq, Dv]
    float* ws_m;    // [n_splits, B*Hq*Lq]
    float* ws_l;
};

__device__ __forceinline__ int heavy_slot(const ssq_decode_args& a, int blk) {
    if (a.pt_dense) return blk;
    if (blk < 64) return __popcll(a.heavy_mask[0] & ((1ull << blk) - 1ull));
    return __popcll(a.heavy_mask[0]) + __popcll(a.heavy_mask[1] & ((1ull << (blk - 64)) - 1ull));
}

template <int VT>
__device__ __forceinline__ void unpack8(const uint4& w, float (&v)[8]) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (VT == SSQ_BF16) {
            v[2 * i] = __uint_as_float(u[i] << 16);
            v[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
        } else {
            v[2 * i] = ssq_f16_to_f32(u[i] & 0xFFFFu);
            v[2 * i + 1] = ssq_f16_to_f32(u[i] >> 16);
        }
    }
}

// load 8 consecutive V elements (16-byte aligned for 16-bit types, 32-byte for fp32)
template <int VT>
__device__ __forceinline__ void load_v8(const void* base, int64_t elem_off, float (&v)[8]) {
    if (VT == SSQ_F32) {
        const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + elem_off);
        const float4 x = p[0], y = p[1];
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
        v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
    } else {
        const uint4 w = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + elem_off);
        unpack8<VT>(w, v);
    }
}

// vector of N floats (N = 1, 2 or a multiple of 4; 4N-byte aligned)
template <int N>
__device__ __forceinline__ void load_vec(const float* __restrict__ src, float (&dst)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            const float4 v = *reinterpret_cast<const float4*>(src + i);
            dst[i] = v.x; dst[i + 1] = v.y; dst[i + 2] = v.z; dst[i + 3] = v.w;
        }
    } else if constexpr (N == 2) {
        const float2 v = *reinterpret_cast<const float2*>(src);
        dst[0] = v.x; dst[1] = v.y;
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) dst[i] = src[i];
    }
}

// LUT[e][r] = sum_d qp[r][blk*BD + d] * C[e][d], e = blk*nc + c: FMA chain over d from the first
// product (triton_kernels.py:381-408).  Each thread loads a batch of kB codewords as vectors, and
// each entry's query sub-vectors as vectors, before the arithmetic: the build then costs a few
// memory / LDS latencies rather than one per element.  Heavy (passthrough) blocks are skipped.
template <int RP, int BD>
__device__ __forceinline__ void build_lut_vec(const ssq_decode_args& a, const float* __restrict__ cent,
                                              const float* __restrict__ qp, float* __restrict__ lut, int tid) {
    constexpr int kB = 64 / BD < 16 ? 64 / BD : 16;
    const int nc = a.n_centroids, D = a.head_dim;
    const int total = a.n_blocks * nc;
    for (int e0 = tid; e0 < total; e0 += kB * kThreads) {
        float c[kB][BD];
#pragma unroll
        for (int kk = 0; kk < kB; ++kk) {
            const int e = e0 + kk * kThreads;
            if (e < total) load_vec<BD>(cent + (int64_t)e * BD, c[kk]);
        }
#pragma unroll
        for (int kk = 0; kk < kB; ++kk) {
            const int e = e0 + kk * kThreads;
            if (e >= total) break;
            const int blk = e / nc;
            if (ssq_is_heavy(a.heavy_mask[0], a.heavy_mask[1], blk)) continue;
            const float* qb = qp + blk * BD;
            float acc[RP];
#pragma unroll
            for (int r = 0; r < RP; ++r) {
                float qv[BD];
                load_vec<BD>(qb + r * D, qv);
                float t = qv[0] * c[kk][0];
#pragma unroll
                for (int d = 1; d < BD; ++d) t = fmaf(qv[d], c[kk][d], t);
                acc[r] = t;
            }
            if constexpr (RP % 4 == 0) {
#pragma unroll
                for (int r = 0; r < RP; r += 4)
                    *reinterpret_cast<float4*>(lut + (size_t)e * RP + r) = make_float4(acc[r], acc[r + 1], acc[r + 2], acc[r + 3]);
            } else {
#pragma unroll
                for (int r = 0; r < RP; ++r) lut[(size_t)e * RP + r] = acc[r];
            }
        }
    }
}

// LUT floats in LDS: none for codebooks past 256 codewords (gathered from global memory)
__host__ __device__ inline size_t lut_floats(const ssq_decode_args& a, int RP) {
    return a.n_centroids > 256 ? 0 : (size_t)a.n_blocks * a.n_centroids * RP;
}

// float offset of the reduction scratch; identical on host and device
__host__ __device__ inline size_t red_offset(const ssq_decode_args& a, int RP, bool has_v) {
    size_t main = lut_floats(a, RP) + (size_t)RP * a.head_dim + (has_v ? (size_t)RP * kTile : 0);
    if (has_v) {
        const int dchunks = a.layout == SSQ_PAGED ? a.value_dim : a.value_dim / 8;
        const size_t epi = (size_t)(kThreads / dchunks) * RP * a.value_dim;
        if (epi > main) main = epi;
    }
    return (main + 3) & ~(size_t)3;
}

template <int RP, bool PAGED, bool HAS_V, int VT>
__global__ __launch_bounds__(kThreads) void k_decode_generic(const DecodeParams p) {
    extern __shared__ __align__(16) float smem[];
    const ssq_decode_args& a = p.a;
    const int tid = threadIdx.x;
    const int lane = tid & (SSQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / SSQ_WAVE);  // wave-uniform: scalar loop control
    const int split = blockIdx.x;
    const int grp = blockIdx.y;
    const int bk = blockIdx.z;
    const int b = bk / a.num_kv_heads;
    const int kv = bk - b * a.num_kv_heads;
    const int nb = a.n_blocks, nc = a.n_centroids, D = a.head_dim, bd = a.block_dim;
    const bool any_heavy = (a.heavy_mask[0] | a.heavy_mask[1]) != 0;
    const int r0 = grp * p.R;
    const int nr = min(p.R, p.rows - r0);
    const int T = PAGED ? min(a.seq_lens[b], a.seq_len) : a.seq_len;
    const int t_begin = split * p.split_len;
    const int t_end = min(T, t_begin + p.split_len);

    // LDS: lut [nb*nc][RP] | qp [RP][D] | ptile [RP][kTile] ... red [2][4][RP] after the
    // larger of that carve-out and the epilogue's [tpar][RP][Dv] output buffer.
    float* lut = smem;
    float* qp = lut + lut_floats(a, RP);
    float* ptile = qp + RP * D;
    float* red = smem + red_offset(a, RP, HAS_V);

    // ---- 1. scaled, permuted query rows (4 elements per thread per pass, their permutation
    // entries and gathers each issued together; indexes clamped so no load sits behind a branch)
    const int64_t* perm = a.perm + (int64_t)kv * a.perm_sh;
    for (int e0 = 0; e0 < RP * D; e0 += 4 * kThreads) {
        int64_t src[4];
        bool ok[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = e0 + k * kThreads + tid;
            src[k] = perm[e < RP * D ? e % D : 0];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = e0 + k * kThreads + tid;
            const int r = e / D;
            ok[k] = e < RP * D && r < nr;
            if (ok[k]) {
                const int row = r0 + r;
                const int g = row / a.q_len, qi = row - g * a.q_len;
                const int h = kv * p.G + g;
                src[k] += (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)qi * a.q_sl;
            }
        }
        float v[4];
        ssq_load_elems(a.q, a.q_dtype, src, v);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = e0 + k * kThreads + tid;
            if (e < RP * D) qp[e] = !ok[k] ? 0.f : a.has_scale ? ssq_round_to(v[k] * a.scale, a.q_dtype) : v[k];
        }
    }
    __syncthreads();

    // ---- 2. LUT build (fp32 FMA chain over the block's dims, dims ascending)
    const float* cent = a.cent + (int64_t)kv * a.cent_sh;
    // vector codeword / query loads need a 16-byte aligned codebook (host-checked: vec_cent)
    // and a 4-aligned head_dim
    const int vb = p.vec_cent ? bd : 0;
    if (p.cw > 1) {
        // no LUT: codewords are gathered per token
    } else if (vb == 1) build_lut_vec<RP, 1>(a, cent, qp, lut, tid);
    else if (vb == 2) build_lut_vec<RP, 2>(a, cent, qp, lut, tid);
    else if (vb == 4) build_lut_vec<RP, 4>(a, cent, qp, lut, tid);
    else if (vb == 8) build_lut_vec<RP, 8>(a, cent, qp, lut, tid);
    else for (int e = tid; e < nb * nc; e += kThreads) {
        const int blk = e / nc;
        if (ssq_is_heavy(a.heavy_mask[0], a.heavy_mask[1], blk)) continue;
        const float* c = cent + (int64_t)e * bd;
        float acc[RP];
#pragma unroll
        for (int r = 0; r < RP; ++r) acc[r] = qp[r * D + blk * bd] * c[0];
        for (int d = 1; d < bd; ++d) {
            const float cd = c[d];
#pragma unroll
            for (int r = 0; r < RP; ++r) acc[r] = fmaf(qp[r * D + blk * bd + d], cd, acc[r]);
        }
#pragma unroll
        for (int r = 0; r < RP; ++r) lut[(size_t)e * RP + r] = acc[r];
    }
    __syncthreads();

    // ---- 3. token tiles
    float m_run[RP], l_thr[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) { m_run[r] = -INFINITY; l_thr[r] = 0.f; }

    // P.V thread mapping
    const int Dv = a.value_dim;
    constexpr int kAccW = PAGED ? 1 : 8;        // dims per thread
    const int dchunks = PAGED ? Dv : Dv / 8;    // threads per token row / per group
    const int tpar = kThreads / dchunks;        // token lanes in parallel
    const int pv_t = tid / dchunks;             // this thread's token lane
    const int pv_d = tid - pv_t * dchunks;      // this thread's dim chunk
    const bool pv_active = pv_t < tpar;
    float acc[RP][kAccW];
#pragma unroll
    for (int r = 0; r < RP; ++r)
#pragma unroll
        for (int j = 0; j < kAccW; ++j) acc[r][j] = 0.f;

    // ---- contiguous layout: the next tile's inputs are loaded into registers while the current
    // tile computes -- this thread's token code words (word-aligned uint8 codes, nb <= 32, no
    // passthrough blocks) and,
    // with 16-bit V (Dv <= 128), the V chunks of its P.V slots.  The loads are unconditional
    // (addresses clamped to the split's last token; those tokens get p = 0), so the compiler's
    // vmcnt waits for the current tile never drain the next one.
    constexpr int kCW = 8, kVC = 16;
    const bool pf_codes = !PAGED && p.word_codes && nb <= 4 * kCW && !any_heavy;
    const bool pf_v = !PAGED && HAS_V && VT != SSQ_F32 && Dv <= 8 * kVC && pv_active;  // nvc <= kVC then
    const int nvc = (kTile + tpar - 1) / tpar;  // P.V slots per thread per tile (token pv_t + k*tpar < kTile)
    uint32_t cwn[kCW];
    uint4 vvn[kVC];
#pragma unroll
    for (int i = 0; i < kCW; ++i) cwn[i] = 0u;
#pragma unroll
    for (int k = 0; k < kVC; ++k) vvn[k] = make_uint4(0u, 0u, 0u, 0u);
    auto prefetch = [&](int t0n) {
        if (pf_codes) {
            const int tc = min(t0n + tid, t_end - 1);
            const uint32_t* w = reinterpret_cast<const uint32_t*>(
                a.codes + (int64_t)b * a.c_sb + (int64_t)kv * a.c_sh + (int64_t)tc * a.c_st);
#pragma unroll
            for (int i = 0; i < kCW; ++i)
                if (i < (nb >> 2)) cwn[i] = w[i];
        }
        if (pf_v) {
            const uint16_t* vb = reinterpret_cast<const uint16_t*>(a.v) + (int64_t)b * a.v_sb + (int64_t)kv * a.v_sh + pv_d * 8;
#pragma unroll
            for (int k = 0; k < kVC; ++k)
                if (k < nvc && pv_t + k * tpar < kTile) {
                    const int tv = min(t0n + pv_t + k * tpar, t_end - 1);
                    vvn[k] = *reinterpret_cast<const uint4*>(vb + (int64_t)tv * a.v_st);
                }
        }
    };
    const int last_t0 = t_end > t_begin ? t_begin + (t_end - 1 - t_begin) / kTile * kTile : t_begin;
    if (t_end > t_begin) prefetch(t_begin);

    for (int t0 = t_begin; t0 < t_end; t0 += kTile) {
        const int t = t0 + tid;
        const bool valid = t < t_end;
        uint32_t cw[kCW];
        uint4 vv[kVC];
#pragma unroll
        for (int i = 0; i < kCW; ++i) cw[i] = cwn[i];
#pragma unroll
        for (int k = 0; k < kVC; ++k) vv[k] = vvn[k];
        prefetch(min(t0 + kTile, last_t0));
        float s[RP];
#pragma unroll
        for (int r = 0; r < RP; ++r) s[r] = 0.f;
        if (valid) {
            int64_t cofs, pt_base;  // code row offset (bytes, or words when packed)
            if (PAGED) {
                const int page = a.block_table[(int64_t)b * a.bt_sb + t / a.page_size];
                const int off = t - (t / a.page_size) * a.page_size;
                cofs = (int64_t)page * a.c_sb + (int64_t)kv * a.c_sh + (int64_t)off * a.c_st;
                pt_base = (int64_t)page * a.pt_sb + (int64_t)kv * a.pt_sh + (int64_t)off * a.pt_st;
            } else {
                cofs = (int64_t)b * a.c_sb + (int64_t)kv * a.c_sh + (int64_t)t * a.c_st;
                pt_base = (int64_t)b * a.pt_sb + (int64_t)kv * a.pt_sh + (int64_t)t * a.pt_st;
            }
            const uint8_t* crow = a.codes + cofs;
            auto add_block = [&](int blk, uint32_t code) {
                if (ssq_is_heavy(a.heavy_mask[0], a.heavy_mask[1], blk)) {
                    const int64_t po = pt_base + (int64_t)heavy_slot(a, blk) * bd;
                    float d_acc[RP];
                    const float x0 = ssq_load_elem(a.pt, a.pt_dtype, po);
#pragma unroll
                    for (int r = 0; r < RP; ++r) d_acc[r] = qp[r * D + blk * bd] * x0;
                    for (int d = 1; d < bd; ++d) {
                        const float xd = ssq_load_elem(a.pt, a.pt_dtype, po + d);
#pragma unroll
                        for (int r = 0; r < RP; ++r) d_acc[r] = fmaf(qp[r * D + blk * bd + d], xd, d_acc[r]);
                    }
#pragma unroll
                    for (int r = 0; r < RP; ++r) s[r] += d_acc[r];
                } else if (p.cw > 1) {
                    // the LUT entry's arithmetic on a gathered codeword: FMA chain over the block's
                    // dims from the first product, then added in block order
                    const uint32_t cc = code < (uint32_t)nc ? code : (uint32_t)(nc - 1);
                    const float* c = cent + ((int64_t)blk * nc + cc) * bd;
                    float e_acc[RP];
                    const float c0 = c[0];
#pragma unroll
                    for (int r = 0; r < RP; ++r) e_acc[r] = qp[r * D + blk * bd] * c0;
                    for (int d = 1; d < bd; ++d) {
                        const float cd = c[d];
#pragma unroll
                        for (int r = 0; r < RP; ++r) e_acc[r] = fmaf(qp[r * D + blk * bd + d], cd, e_acc[r]);
                    }
#pragma unroll
                    for (int r = 0; r < RP; ++r) s[r] += e_acc[r];
                } else {
                    const int cc = (int)code < nc ? (int)code : nc - 1;
                    const float* e = lut + ((size_t)blk * nc + cc) * RP;
                    if (RP % 4 == 0) {
#pragma unroll
                        for (int r = 0; r < RP; r += 4) {
                            const float4 v = *reinterpret_cast<const float4*>(e + r);
                            s[r] += v.x; s[r + 1] += v.y; s[r + 2] += v.z; s[r + 3] += v.w;
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < RP; ++r) s[r] += e[r];
                    }
                }
            };
            if (p.cw > 1 && bd <= 4) {
                // 16- / 32-bit codes (code strides count elements of that width), codewords of at most
                // 4 dims: per batch of 8 blocks the codes are loaded together, then the codewords,
                // then the blocks are added in order (the arithmetic of add_block; two memory round
                // trips per batch instead of two per block)
                constexpr int kBat = 8;
                for (int b0 = 0; b0 < nb; b0 += kBat) {
                    uint32_t code[kBat];
#pragma unroll
                    for (int k = 0; k < kBat; ++k)
                        code[k] = b0 + k < nb ? ssq_load_code(a.codes, p.cw, cofs + b0 + k) : 0u;
                    float cv[kBat][4];
#pragma unroll
                    for (int k = 0; k < kBat; ++k) {
                        const uint32_t cc = code[k] < (uint32_t)nc ? code[k] : (uint32_t)(nc - 1);
                        const float* c = cent + ((int64_t)min(b0 + k, nb - 1) * nc + cc) * bd;
                        if (bd == 4 && p.vec_cent) {  // one 16-byte load (the codebook is 16-byte aligned)
                            const float4 v4 = *reinterpret_cast<const float4*>(c);
                            cv[k][0] = v4.x; cv[k][1] = v4.y; cv[k][2] = v4.z; cv[k][3] = v4.w;
                        } else if (bd == 2 && p.vec_cent) {
                            const float2 v2 = *reinterpret_cast<const float2*>(c);
                            cv[k][0] = v2.x; cv[k][1] = v2.y; cv[k][2] = 0.f; cv[k][3] = 0.f;
                        } else {
#pragma unroll
                            for (int d = 0; d < 4; ++d) cv[k][d] = d < bd ? c[d] : 0.f;
                        }
                    }
#pragma unroll
                    for (int k = 0; k < kBat; ++k) {
                        const int blk = b0 + k;
                        if (blk >= nb) break;
                        if (ssq_is_heavy(a.heavy_mask[0], a.heavy_mask[1], blk)) {
                            add_block(blk, code[k]);
                            continue;
                        }
                        float e_acc[RP];
#pragma unroll
                        for (int r = 0; r < RP; ++r) e_acc[r] = qp[r * D + blk * bd] * cv[k][0];
#pragma unroll
                        for (int d = 1; d < 4; ++d) {
                            if (d < bd) {
#pragma unroll
                                for (int r = 0; r < RP; ++r) e_acc[r] = fmaf(qp[r * D + blk * bd + d], cv[k][d], e_acc[r]);
                            }
                        }
#pragma unroll
                        for (int r = 0; r < RP; ++r) s[r] += e_acc[r];
                    }
                }
            } else if (p.cw > 1) {  // 16- / 32-bit codes, wider codewords: block by block
                for (int blk = 0; blk < nb; ++blk) add_block(blk, ssq_load_code(a.codes, p.cw, cofs + blk));
            } else if (a.code_bits) {  // sub-byte codes packed into uint32 words
                const uint32_t* w = reinterpret_cast<const uint32_t*>(a.codes) + cofs;
                const int bits = a.code_bits, vpe = 32 / bits;
                const uint32_t msk = (1u << bits) - 1u;
                for (int pi = 0, blk = 0; blk < nb; ++pi) {
                    const uint32_t word = w[pi];
                    for (int v = 0; v < vpe && blk < nb; ++v, ++blk) add_block(blk, (word >> (v * bits)) & msk);
                }
            } else if (pf_codes) {
                // LUT gathers 8 blocks at a time, summed in block order
#pragma unroll
                for (int w0 = 0; w0 < kCW; w0 += 2) {
                    if (w0 < (nb >> 2)) {
                        constexpr int NV = RP >= 4 ? RP / 4 : 1;
                        float4 ev[8][NV];
#pragma unroll
                        for (int k = 0; k < 8; ++k) {
                            const int blk = 4 * w0 + k;
                            const uint32_t word = cw[w0 + (k >> 2)];
                            const int code = (int)((word >> (8 * (k & 3))) & 0xFFu);
                            const int cc = code < nc ? code : nc - 1;
                            const float* e = lut + ((size_t)blk * nc + cc) * RP;
                            if (blk < nb) {
                                if (RP >= 4) {
#pragma unroll
                                    for (int j = 0; j < NV; ++j) ev[k][j] = *reinterpret_cast<const float4*>(e + 4 * j);
                                } else if (RP == 2) {
                                    const float2 v2 = *reinterpret_cast<const float2*>(e);
                                    ev[k][0] = make_float4(v2.x, v2.y, 0.f, 0.f);
                                } else {
                                    ev[k][0] = make_float4(e[0], 0.f, 0.f, 0.f);
                                }
                            }
                        }
#pragma unroll
                        for (int k = 0; k < 8; ++k) {
                            if (4 * w0 + k < nb) {
                                if (RP >= 4) {
#pragma unroll
                                    for (int j = 0; j < NV; ++j) {
                                        s[4 * j] += ev[k][j].x; s[4 * j + 1] += ev[k][j].y;
                                        s[4 * j + 2] += ev[k][j].z; s[4 * j + 3] += ev[k][j].w;
                                    }
                                } else if (RP == 2) {
                                    s[0] += ev[k][0].x; s[1] += ev[k][0].y;
                                } else {
                                    s[0] += ev[k][0].x;
                                }
                            }
                        }
                    }
                }
            } else if (p.word_codes) {
                const uint32_t* w = reinterpret_cast<const uint32_t*>(crow);
                for (int wi = 0; wi < (nb >> 2); ++wi) {
                    const uint32_t word = w[wi];
                    add_block(4 * wi + 0, word & 0xFFu);
                    add_block(4 * wi + 1, (word >> 8) & 0xFFu);
                    add_block(4 * wi + 2, (word >> 16) & 0xFFu);
                    add_block(4 * wi + 3, word >> 24);
                }
            } else {
                for (int blk = 0; blk < nb; ++blk) add_block(blk, crow[blk]);
            }
            if (a.mask) {  // every row's load issued before any is added (rows past nr read row 0)
                float mk[RP];
#pragma unroll
                for (int r = 0; r < RP; ++r) {
                    const int row = r0 + (r < nr ? r : 0);
                    const int g = row / a.q_len, qi = row - g * a.q_len;
                    const int h = kv * p.G + g;
                    mk[r] = a.mask[(int64_t)b * a.m_sb + (int64_t)h * a.m_sh + (int64_t)qi * a.m_sl + (int64_t)t * a.m_st];
                }
#pragma unroll
                for (int r = 0; r < RP; ++r)
                    if (r < nr) s[r] += mk[r];
            }
            if (a.scores) {
#pragma unroll
                for (int r = 0; r < RP; ++r) {
                    if (r < nr) {
                        const int row = r0 + r;
                        const int g = row / a.q_len, qi = row - g * a.q_len;
                        const int h = kv * p.G + g;
                        a.scores[(int64_t)b * a.s_sb + (int64_t)h * a.s_sh + (int64_t)qi * a.s_sl + t] = s[r];
                    }
                }
            }
        }
        if (!HAS_V) continue;

        // online softmax over the tile
#pragma unroll
        for (int r = 0; r < RP; ++r) {
            const float v = ssq_wave_max(valid ? s[r] : -INFINITY);
            if (lane == 0) red[wave * RP + r] = v;
        }
        __syncthreads();
        float alpha[RP];
#pragma unroll
        for (int r = 0; r < RP; ++r) {
            float tm = red[r];
#pragma unroll
            for (int w = 1; w < kThreads / SSQ_WAVE; ++w) tm = fmaxf(tm, red[w * RP + r]);
            const float mn = fmaxf(m_run[r], tm);
            alpha[r] = (mn == -INFINITY) ? 1.f : __expf(m_run[r] - mn);
            m_run[r] = mn;
            const float pr = (valid && mn != -INFINITY) ? __expf(s[r] - mn) : 0.f;
            l_thr[r] = l_thr[r] * alpha[r] + pr;
            ptile[r * kTile + tid] = pr;
        }
        __syncthreads();

        // P.V
        const int nt = min(kTile, t_end - t0);
#pragma unroll
        for (int r = 0; r < RP; ++r)
#pragma unroll
            for (int j = 0; j < kAccW; ++j) acc[r][j] *= alpha[r];
        if (pv_active) {
            if (pf_v) {
#pragma unroll
                for (int k = 0; k < kVC; ++k) {
                    const int tt = pv_t + k * tpar;
                    if (k < nvc && tt < kTile) {
                        float v[8];
                        unpack8<VT>(vv[k], v);
#pragma unroll
                        for (int r = 0; r < RP; ++r) {
                            const float pr = ptile[r * kTile + tt];
#pragma unroll
                            for (int j = 0; j < 8; ++j) acc[r][j] = fmaf(pr, v[j], acc[r][j]);
                        }
                    }
                }
            } else if (!PAGED) {
                const int64_t vbase = (int64_t)b * a.v_sb + (int64_t)kv * a.v_sh + pv_d * 8;
                for (int tt = pv_t; tt < nt; tt += tpar) {
                    float v[8];
                    load_v8<VT>(a.v, vbase + (int64_t)(t0 + tt) * a.v_st, v);
#pragma unroll
                    for (int r = 0; r < RP; ++r) {
                        const float pr = ptile[r * kTile + tt];
#pragma unroll
                        for (int j = 0; j < 8; ++j) acc[r][j] = fmaf(pr, v[j], acc[r][j]);
                    }
                }
            } else {
                // V pages [P, Hkv, Dv, page]: 8 consecutive tokens of one dim per load
                const int nchunks = (nt + 7) >> 3;
                for (int ch = pv_t; ch < nchunks; ch += tpar) {
                    const int tt = ch * 8;
                    const int t = t0 + tt;
                    const int page = a.block_table[(int64_t)b * a.bt_sb + t / a.page_size];
                    const int off = t - (t / a.page_size) * a.page_size;
                    float v[8];
                    load_v8<VT>(a.v, (int64_t)page * a.v_sb + (int64_t)kv * a.v_sh + (int64_t)pv_d * a.v_st + off, v);
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        if (tt + j >= nt) v[j] = 0.f;  // tokens past the end: p = 0 and V unwritten
#pragma unroll
                    for (int r = 0; r < RP; ++r) {
                        const float4 p0 = *reinterpret_cast<const float4*>(ptile + r * kTile + tt);
                        const float4 p1 = *reinterpret_cast<const float4*>(ptile + r * kTile + tt + 4);
                        float x = acc[r][0];
                        x = fmaf(p0.x, v[0], x); x = fmaf(p0.y, v[1], x);
                        x = fmaf(p0.z, v[2], x); x = fmaf(p0.w, v[3], x);
                        x = fmaf(p1.x, v[4], x); x = fmaf(p1.y, v[5], x);
                        x = fmaf(p1.z, v[6], x); x = fmaf(p1.w, v[7], x);
                        acc[r][0] = x;
                    }
                }
            }
        }
        __syncthreads();
    }
    if (!HAS_V) return;

    // ---- 4. epilogue: reduce l over threads, o over token lanes
    float* red2 = red + (kThreads / SSQ_WAVE) * RP;
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        const float v = ssq_wave_sum(l_thr[r]);
        if (lane == 0) red2[wave * RP + r] = v;
    }
    float* obuf = smem;  // reuses the LUT region: [tpar][RP][Dv]
    if (pv_active) {
#pragma unroll
        for (int r = 0; r < RP; ++r)
#pragma unroll
            for (int j = 0; j < kAccW; ++j) obuf[((size_t)pv_t * RP + r) * Dv + pv_d * kAccW + j] = acc[r][j];
    }
    __syncthreads();
    const int n_rows_all = a.batch * a.num_q_heads * a.q_len;
    for (int e = tid; e < nr * Dv; e += kThreads) {
        const int r = e / Dv, dv = e - r * Dv;
        float l = 0.f;
        for (int w = 0; w < kThreads / SSQ_WAVE; ++w) l += red2[w * RP + r];
        float o = 0.f;
        for (int g2 = 0; g2 < tpar; ++g2) o += obuf[((size_t)g2 * RP + r) * Dv + dv];
        float m = 0.f;
#pragma unroll
        for (int rr = 0; rr < RP; ++rr)
            if (rr == r) m = m_run[rr];
        const int row = r0 + r;
        const int g = row / a.q_len, qi = row - g * a.q_len;
        const int h = kv * p.G + g;
        const int rid = (b * a.num_q_heads + h) * a.q_len + qi;
        if (p.n_splits == 1) {
            ssq_store_elem(a.out, a.v_dtype, (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)qi * a.o_sl + dv, o / l);
            if (a.lse && dv == 0) a.lse[rid] = m + logf(l);
        } else {
            p.ws_o[((size_t)split * n_rows_all + rid) * Dv + dv] = o;
            if (dv == 0) {
                p.ws_m[(size_t)split * n_rows_all + rid] = m;
                p.ws_l[(size_t)split * n_rows_all + rid] = l;
            }
        }
    }
}

// Combine split partials: out = sum_s o_s e^{m_s-M} / sum_s l_s e^{m_s-M}, lse = M + log L.
// One wave per query row, kMergeRows rows per workgroup.  Lane j merges value dims j, j + 64, ...;
// every lane loads the row's (m_s, l_s) and its dims' o_s for up to kMergeSplits splits before
// using any of them, so a merge of that many splits costs one memory round trip (more splits take
// further passes, merged online).  No LDS and no workgroup barrier.
constexpr int kMergeRows = 4;
constexpr int kMergeSplits = 16;
constexpr int kMergeDims = 4;  // value dims per lane per pass: 256 per wave

__global__ __launch_bounds__(kMergeRows * SSQ_WAVE) void k_merge(const ssq_decode_args a, int n_splits,
                                                                  const float* ws_o, const float* ws_m,
                                                                  const float* ws_l) {
    const int lane = threadIdx.x & (SSQ_WAVE - 1);
    const int n_rows_all = a.batch * a.num_q_heads * a.q_len;
    const int rid = blockIdx.x * kMergeRows + (int)(threadIdx.x / SSQ_WAVE);
    if (rid >= n_rows_all) return;  // whole waves
    const int qi = rid % a.q_len;
    const int h = (rid / a.q_len) % a.num_q_heads;
    const int b = rid / (a.q_len * a.num_q_heads);
    const int Dv = a.value_dim;
    const size_t mstep = (size_t)n_rows_all;       // between splits in ws_m / ws_l
    const size_t ostep = (size_t)n_rows_all * Dv;  // between splits in ws_o
    float M = -INFINITY, L = 0.f;
    for (int d0 = 0; d0 < Dv; d0 += kMergeDims * SSQ_WAVE) {
        float Mr = -INFINITY, Lr = 0.f;
        float o[kMergeDims];
#pragma unroll
        for (int k = 0; k < kMergeDims; ++k) o[k] = 0.f;
        for (int c0 = 0; c0 < n_splits; c0 += kMergeSplits) {
            float mv[kMergeSplits], lv[kMergeSplits], ov[kMergeSplits][kMergeDims];
#pragma unroll
            for (int i = 0; i < kMergeSplits; ++i) {
                mv[i] = -INFINITY;
                lv[i] = 0.f;
#pragma unroll
                for (int k = 0; k < kMergeDims; ++k) ov[i][k] = 0.f;
                if (c0 + i < n_splits) {  // uniform
                    const size_t s = (size_t)(c0 + i);
                    mv[i] = ws_m[s * mstep + rid];
                    lv[i] = ws_l[s * mstep + rid];
#pragma unroll
                    for (int k = 0; k < kMergeDims; ++k)
                        if (d0 + k * SSQ_WAVE < Dv)  // uniform; the lane's dim is clamped
                            ov[i][k] = ws_o[s * ostep + (size_t)rid * Dv + min(d0 + k * SSQ_WAVE + lane, Dv - 1)];
                }
            }
            float Mc = Mr;
#pragma unroll
            for (int i = 0; i < kMergeSplits; ++i) Mc = fmaxf(Mc, mv[i]);
            const float f = Mr == -INFINITY ? 0.f : __expf(Mr - Mc);  // earlier passes, rescaled
            Lr *= f;
#pragma unroll
            for (int k = 0; k < kMergeDims; ++k) o[k] *= f;
#pragma unroll
            for (int i = 0; i < kMergeSplits; ++i) {
                const float w = mv[i] == -INFINITY ? 0.f : __expf(mv[i] - Mc);
                Lr += lv[i] * w;
#pragma unroll
                for (int k = 0; k < kMergeDims; ++k) o[k] += ov[i][k] * w;
            }
            Mr = Mc;
        }
#pragma unroll
        for (int k = 0; k < kMergeDims; ++k) {
            const int dv = d0 + k * SSQ_WAVE + lane;
            if (dv < Dv)
                ssq_store_elem(a.out, a.v_dtype, (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)qi * a.o_sl + dv,
                               o[k] / Lr);
        }
        M = Mr;
        L = Lr;
    }
    if (a.lse && lane == 0) a.lse[rid] = M + logf(L);
}

static int launch_merge(const ssq_decode_args& a, int n_splits, const float* ws_o, const float* ws_m,
                        const float* ws_l, hipStream_t st) {
    const int n_rows_all = a.batch * a.num_q_heads * a.q_len;
    hipLaunchKernelGGL(k_merge, dim3((unsigned)((n_rows_all + kMergeRows - 1) / kMergeRows)),
                       dim3(kMergeRows * SSQ_WAVE), 0, st, a, n_splits, ws_o, ws_m, ws_l);
    return ssq_check_hip(hipGetLastError(), "k_merge launch");
}

// --------------------------------------------------------------------------
// host side
// --------------------------------------------------------------------------
struct Plan {
    int G, rows, R, RP, n_groups, split_len, n_splits;
    size_t smem;
    size_t ws_bytes;
    bool has_v;
};

int pow2_at_least(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

size_t smem_bytes(const ssq_decode_args& a, int RP, bool has_v) {
    return (red_offset(a, RP, has_v) + 2 * (kThreads / SSQ_WAVE) * RP) * sizeof(float);
}

constexpr size_t kMaxSmem = 160 * 1024;

int make_plan(const ssq_decode_args& a, Plan& pl) {
    pl.has_v = a.v != nullptr;
    pl.G = a.num_q_heads / a.num_kv_heads;
    pl.rows = pl.G * a.q_len;
    int R = pl.rows < kMaxRows ? pl.rows : kMaxRows;
    for (; R >= 1; --R) {
        if (smem_bytes(a, pow2_at_least(R), pl.has_v) <= kMaxSmem) break;
    }
    SSQ_UNSUPPORTED(R >= 1, "codebook too large for LDS: n_blocks*n_centroids=%d", a.n_blocks * a.n_centroids);
    pl.R = R;
    pl.RP = pow2_at_least(R);
    pl.n_groups = (pl.rows + R - 1) / R;
    pl.smem = smem_bytes(a, pl.RP, pl.has_v);
    const int units = a.batch * a.num_kv_heads * pl.n_groups;
    const int tiles = (a.seq_len + kTile - 1) / kTile;
    // one round of workgroups: as many as the device runs at once at this LDS footprint
    // (each split rebuilds the LUT, so a second round costs more than it hides)
    const int per_cu = pl.smem > 0 ? (int)(kMaxSmem / pl.smem) : 1;
    const int slots = ssq_device_cus() * (per_cu < 1 ? 1 : per_cu > 2 ? 2 : per_cu);
    int splits = a.num_splits > 0 ? a.num_splits : (slots + units - 1) / units;
    if (splits > tiles) splits = tiles;
    if (splits < 1) splits = 1;
    const int tiles_per_split = (tiles + splits - 1) / splits;
    pl.split_len = tiles_per_split * kTile;
    pl.n_splits = (a.seq_len + pl.split_len - 1) / pl.split_len;
    if (pl.n_splits < 1) pl.n_splits = 1;
    const size_t n_rows_all = (size_t)a.batch * a.num_q_heads * a.q_len;
    pl.ws_bytes = (pl.has_v && pl.n_splits > 1) ? (size_t)pl.n_splits * n_rows_all * (a.value_dim + 2) * 4 : 0;
    return SSQ_OK;
}

int validate(const ssq_decode_args* a, bool need_v) {
    if (!a) return ssq_fail(SSQ_ERR_INVALID, "args is NULL");
    if (a->struct_size != sizeof(ssq_decode_args))
        return ssq_fail(SSQ_ERR_ABI, "ssq_decode_args size %u != library's %zu", a->struct_size, sizeof(ssq_decode_args));
    SSQ_REQUIRE(a->q && a->perm && a->cent && a->codes, "q, perm, cent and codes must be non-NULL");
    SSQ_REQUIRE(a->batch >= 1 && a->num_q_heads >= 1 && a->q_len >= 1 && a->num_kv_heads >= 1, "empty batch/heads");
    SSQ_REQUIRE(a->num_q_heads % a->num_kv_heads == 0, "Query head count must be divisible by kv-head count.");
    SSQ_REQUIRE(a->block_dim >= 1 && a->head_dim % a->block_dim == 0, "head_dim must be divisible by block_dim");
    SSQ_REQUIRE(a->n_blocks == a->head_dim / a->block_dim, "n_blocks != head_dim / block_dim");
    SSQ_REQUIRE(a->head_dim <= 1024, "head_dim > 1024");
    SSQ_REQUIRE(a->n_centroids >= 1 && a->n_centroids <= kMaxCentroids, "n_centroids must be in [1, %d]", kMaxCentroids);
    SSQ_REQUIRE(a->n_blocks <= 128, "n_blocks > 128");
    SSQ_REQUIRE(a->code_bits >= 0 && a->code_bits <= 8, "code_bits must be 0 (uint8) or 1..8 (packed)");
    SSQ_REQUIRE(a->n_centroids <= 256 || a->code_bits == 0,
                "n_centroids=%d takes 16- or 32-bit codes (code_bits 0)", a->n_centroids);
    if (a->n_centroids > 256) {
        const int cw = ssq_code_width(a->n_centroids);
        SSQ_REQUIRE((uintptr_t)a->codes % cw == 0, "%d-bit codes must be %d-byte aligned", 8 * cw, cw);
    }
    if (a->code_bits) {
        SSQ_REQUIRE(a->n_centroids <= (1 << a->code_bits), "n_centroids=%d needs more than %d-bit codes",
                    a->n_centroids, a->code_bits);
        SSQ_REQUIRE((uintptr_t)a->codes % 4 == 0, "packed codes must be 4-byte aligned");
    }
    SSQ_REQUIRE(a->q_dtype >= SSQ_F32 && a->q_dtype <= SSQ_F16, "bad q_dtype");
    SSQ_REQUIRE(a->seq_len >= 0, "negative seq_len");
    const bool any_heavy = a->heavy_mask[0] || a->heavy_mask[1];
    SSQ_REQUIRE(!any_heavy || a->pt, "Mixed-precision quantized keys are missing passthrough values.");
    if (any_heavy) SSQ_REQUIRE(a->pt_dtype >= SSQ_F32 && a->pt_dtype <= SSQ_F16, "bad pt_dtype");
    SSQ_REQUIRE(a->layout == SSQ_CONTIGUOUS || a->layout == SSQ_PAGED, "bad layout");
    if (a->layout == SSQ_PAGED) {
        SSQ_REQUIRE(a->block_table && a->seq_lens, "paged layout needs block_table and seq_lens");
        SSQ_REQUIRE(a->page_size >= 8 && a->page_size <= kTile && kTile % a->page_size == 0,
                    "page_size must divide %d and be >= 8", kTile);
    }
    if (need_v) {
        SSQ_REQUIRE(a->v && a->out, "decode needs v and out");
        SSQ_REQUIRE(a->v_dtype >= SSQ_F32 && a->v_dtype <= SSQ_F16, "bad v_dtype");
        SSQ_REQUIRE(a->value_dim >= 8 && a->value_dim % 8 == 0 && a->value_dim <= kThreads &&
                        (a->layout == SSQ_PAGED ? kThreads % a->value_dim == 0 : kThreads % (a->value_dim / 8) == 0),
                    "unsupported value_dim %d", a->value_dim);
        SSQ_REQUIRE(a->layout == SSQ_CONTIGUOUS || a->page_size % 8 == 0, "paged V needs page_size % 8 == 0");
    }
    return SSQ_OK;
}

template <int RP, bool PAGED, bool HAS_V, int VT>
int launch_t(const DecodeParams& dp, const Plan& pl, hipStream_t st) {
    auto kern = k_decode_generic<RP, PAGED, HAS_V, VT>;
    int rc = ssq_allow_lds((const void*)kern, (int)kMaxSmem, "hipFuncSetAttribute(decode)");
    if (rc) return rc;
    dim3 grid(pl.n_splits, pl.n_groups, dp.a.batch * dp.a.num_kv_heads);
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), pl.smem, st, dp);
    return ssq_check_hip(hipGetLastError(), "k_decode_generic launch");
}

template <int RP, bool PAGED, bool HAS_V>
int launch_vt(const DecodeParams& dp, const Plan& pl, hipStream_t st) {
    if (!HAS_V) return launch_t<RP, PAGED, HAS_V, SSQ_BF16>(dp, pl, st);
    switch (dp.a.v_dtype) {
        case SSQ_BF16: return launch_t<RP, PAGED, HAS_V, SSQ_BF16>(dp, pl, st);
        case SSQ_F16: return launch_t<RP, PAGED, HAS_V, SSQ_F16>(dp, pl, st);
        default: return launch_t<RP, PAGED, HAS_V, SSQ_F32>(dp, pl, st);
    }
}

template <int RP>
int launch_rp(const DecodeParams& dp, const Plan& pl, hipStream_t st) {
    const bool paged = dp.a.layout == SSQ_PAGED;
    if (paged) return pl.has_v ? launch_vt<RP, true, true>(dp, pl, st) : launch_vt<RP, true, false>(dp, pl, st);
    return pl.has_v ? launch_vt<RP, false, true>(dp, pl, st) : launch_vt<RP, false, false>(dp, pl, st);
}

int run_generic(const ssq_decode_args* a, void* workspace, size_t ws_bytes, hipStream_t st) {
    Plan pl;
    int rc = make_plan(*a, pl);
    if (rc) return rc;
    if (a->seq_len == 0) return ssq_fail(SSQ_ERR_INVALID, "seq_len == 0: softmax over an empty context");
    SSQ_REQUIRE(ws_bytes >= pl.ws_bytes, "workspace too small: %zu < %zu bytes", ws_bytes, pl.ws_bytes);
    SSQ_REQUIRE(pl.ws_bytes == 0 || workspace, "workspace is NULL");
    DecodeParams dp;
    dp.a = *a;
    dp.G = pl.G;
    dp.rows = pl.rows;
    dp.R = pl.R;
    dp.split_len = pl.split_len;
    dp.n_splits = pl.n_splits;
    dp.cw = ssq_code_width(a->n_centroids);
    const bool aligned = dp.cw == 1 && a->code_bits == 0 && ((uintptr_t)a->codes % 4 == 0) && a->n_blocks % 4 == 0 &&
                         a->c_st % 4 == 0 && a->c_sh % 4 == 0 && a->c_sb % 4 == 0;
    dp.word_codes = aligned ? 1 : 0;
    dp.vec_cent = ((uintptr_t)a->cent % 16 == 0 && (a->cent_sh * 4) % 16 == 0 && a->head_dim % 4 == 0 &&
                   (a->n_blocks * a->n_centroids) % 4 == 0) ? 1 : 0;  // qp (after the LUT) 16-byte aligned
    const size_t n_rows_all = (size_t)a->batch * a->num_q_heads * a->q_len;
    float* ws = reinterpret_cast<float*>(workspace);
    dp.ws_o = ws;
    dp.ws_m = ws ? ws + (size_t)pl.n_splits * n_rows_all * a->value_dim : nullptr;
    dp.ws_l = ws ? dp.ws_m + (size_t)pl.n_splits * n_rows_all : nullptr;
    if (pl.has_v) {
        // 16-byte vector loads of V
        const int esz = a->v_dtype == SSQ_F32 ? 4 : 2;
        SSQ_REQUIRE((uintptr_t)a->v % 16 == 0 && (a->v_sb * esz) % 16 == 0 && (a->v_sh * esz) % 16 == 0 &&
                        (a->v_st * esz) % 16 == 0,
                    "V must be 16-byte aligned with 16-byte aligned strides");
    }
    switch (pl.RP) {
        case 1: rc = launch_rp<1>(dp, pl, st); break;
        case 2: rc = launch_rp<2>(dp, pl, st); break;
        case 4: rc = launch_rp<4>(dp, pl, st); break;
        default: rc = launch_rp<8>(dp, pl, st); break;
    }
    if (rc) return rc;
    if (pl.has_v && pl.n_splits > 1) {
        rc = launch_merge(*a, pl.n_splits, dp.ws_o, dp.ws_m, dp.ws_l, st);
    }
    return rc;
}

}  // namespace

// Launches the split merge (shared with the MFMA decode kernel).
int ssq_launch_merge(const ssq_decode_args& a, int n_splits, const float* ws_o, const float* ws_m,
                     const float* ws_l, hipStream_t st) {
    return launch_merge(a, n_splits, ws_o, ws_m, ws_l, st);
}

int ssq_decode_mfma_supported(const ssq_decode_args* a);
size_t ssq_decode_mfma_workspace(const ssq_decode_args* a);
int ssq_decode_mfma(const ssq_decode_args* a, void* workspace, size_t ws_bytes, hipStream_t st);
int ssq_decode_contig_supported(const ssq_decode_args* a);
size_t ssq_decode_contig_workspace(const ssq_decode_args* a);
int ssq_decode_contig(const ssq_decode_args* a, void* workspace, size_t ws_bytes, hipStream_t st);

namespace {
// kernel choice: 2 = MFMA paged, 3 = MFMA contiguous, 1 = generic; 0 picks the first that serves
int pick_kernel(const ssq_decode_args* a) {
    if (a->kernel == 4) return 2;  // the paged MFMA path, with its 4x4-MFMA-scores kernel forced
    if (a->kernel != 0) return a->kernel;
    // (the MFMA kernel's plan takes scores-only problems on contiguous rows past head_dim 64)
    if (ssq_decode_mfma_supported(a)) return 2;
    // scores only or decode: the contiguous MFMA kernel where it applies (its 4x4-MFMA scores need no
    // per-workgroup LUT: config-2 scores 11.9 us against the LUT kernel's 18.3 us), else the generic one
    if (ssq_decode_contig_supported(a)) return 3;
    return 1;
}
}  // namespace

extern "C" size_t ssq_decode_workspace_size(const ssq_decode_args* a) {
    if (validate(a, a && a->v != nullptr) != SSQ_OK) return 0;
    const int k = pick_kernel(a);
    if (k == 2 && a->v && ssq_decode_mfma_supported(a)) return ssq_decode_mfma_workspace(a);
    if (k == 3 && ssq_decode_contig_supported(a)) return ssq_decode_contig_workspace(a);
    Plan pl;
    if (make_plan(*a, pl) != SSQ_OK) return 0;
    return pl.ws_bytes;
}

extern "C" int ssq_decode(const ssq_decode_args* a, void* workspace, size_t workspace_bytes, void* stream) {
    int rc = validate(a, true);
    if (rc) return rc;
    const int k = pick_kernel(a);
    if (k == 2) {
        SSQ_UNSUPPORTED(ssq_decode_mfma_supported(a), "MFMA decode kernel does not support this problem");
        return ssq_decode_mfma(a, workspace, workspace_bytes, (hipStream_t)stream);
    }
    if (k == 3) {
        SSQ_UNSUPPORTED(ssq_decode_contig_supported(a), "contiguous MFMA kernel does not support this problem");
        return ssq_decode_contig(a, workspace, workspace_bytes, (hipStream_t)stream);
    }
    return run_generic(a, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int ssq_attention_scores(const ssq_decode_args* a, void* stream) {
    int rc = validate(a, false);
    if (rc) return rc;
    SSQ_REQUIRE(a->v == nullptr && a->scores != nullptr, "scores-only call needs v == NULL and scores != NULL");
    if (a->seq_len == 0) return SSQ_OK;
    const int k = pick_kernel(a);
    if (k == 2) {
        SSQ_UNSUPPORTED(ssq_decode_mfma_supported(a), "MFMA LUT kernel does not support this scores-only problem");
        return ssq_decode_mfma(a, nullptr, 0, (hipStream_t)stream);
    }
    if (k == 3) {
        SSQ_UNSUPPORTED(ssq_decode_contig_supported(a), "contiguous MFMA kernel does not support this problem");
        return ssq_decode_contig(a, nullptr, 0, (hipStream_t)stream);
    }
    return run_generic(a, nullptr, 0, (hipStream_t)stream);
}
