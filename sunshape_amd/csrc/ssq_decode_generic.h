// VQ-key decode attention, the generic kernel: LUT build in LDS + code gather-sum + online
// softmax + P.V.  The kernel template and its launchers; the host plan is in ssq_decode.hip, which
// instantiates the byte / packed / 32-bit-code variants, and ssq_decode_generic_w16.hip the 16-bit
// code ones (compiled in parallel).
//
// Any head grouping, block_dim, contiguous or paged layout.
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
#pragma once

#include "ssq_common.h"

#include <math.h>

#include <type_traits>

// parameters of k_decode_generic (shared by its instantiation units)
struct SsqGenericParams {
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

// launch shape of k_decode_generic
struct SsqGenericLaunch {
    int RP;        // query rows per workgroup, rounded up to a power of two
    int n_splits;  // grid.x
    int n_groups;  // grid.y (row groups); grid.z = batch * KV heads
    size_t smem;   // dynamic LDS bytes
    bool has_v;
};

namespace {

constexpr int kThreads = 256;
constexpr int kTile = 256;   // tokens per main-loop iteration
constexpr int kMaxRows = 8;  // query rows per workgroup (LUT is [nb][nc][RP])
constexpr size_t kMaxSmem = 160 * 1024;

using DecodeParams = SsqGenericParams;

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

// 8 consecutive V elements as loaded (unpacked by unpack_v8), so several loads can be in flight
// before any is used
template <int VT>
struct VRaw8 {
    uint4 w[VT == SSQ_F32 ? 2 : 1];
};

typedef unsigned int ssq_v4u __attribute__((ext_vector_type(4)));

// a 16-byte load that streams past the caches (NT) or a plain one
template <bool NT>
__device__ __forceinline__ uint4 ld16g(const void* p) {
    if constexpr (NT) {
        const ssq_v4u v = __builtin_nontemporal_load(reinterpret_cast<const ssq_v4u*>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *reinterpret_cast<const uint4*>(p);
    }
}

template <int VT, bool NT = false>
__device__ __forceinline__ VRaw8<VT> load_v8_raw(const void* base, int64_t elem_off) {
    VRaw8<VT> r;
    if constexpr (VT == SSQ_F32) {
        const float* q = reinterpret_cast<const float*>(base) + elem_off;
        r.w[0] = ld16g<NT>(q);
        r.w[1] = ld16g<NT>(q + 4);
    } else {
        r.w[0] = ld16g<NT>(reinterpret_cast<const uint16_t*>(base) + elem_off);
    }
    return r;
}

template <int VT>
__device__ __forceinline__ void unpack_v8(const VRaw8<VT>& r, float (&v)[8]) {
    if constexpr (VT == SSQ_F32) {
        v[0] = __uint_as_float(r.w[0].x); v[1] = __uint_as_float(r.w[0].y);
        v[2] = __uint_as_float(r.w[0].z); v[3] = __uint_as_float(r.w[0].w);
        v[4] = __uint_as_float(r.w[1].x); v[5] = __uint_as_float(r.w[1].y);
        v[6] = __uint_as_float(r.w[1].z); v[7] = __uint_as_float(r.w[1].w);
    } else {
        unpack8<VT>(r.w[0], v);
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
    size_t main = lut_floats(a, RP) + (size_t)RP * a.head_dim +
                  (has_v ? (size_t)RP * kTile + (a.layout == SSQ_PAGED ? kTile : 0) : 0);
    if (has_v) {
        const int dchunks = a.layout == SSQ_PAGED ? a.value_dim : a.value_dim / 8;
        const size_t epi = (size_t)(kThreads / dchunks) * RP * a.value_dim;
        if (epi > main) main = epi;
    }
    return (main + 3) & ~(size_t)3;
}

// W16: 16-bit codes in 16-byte aligned rows of a multiple of 8 blocks (at most 64), codewords of 2
// or 4 dims in a 16-byte aligned codebook (host-checked); those variants keep no other code path.
template <int RP, bool PAGED, bool HAS_V, int VT, bool W16>
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

    // LDS: lut [nb*nc][RP] | qp [RP][D] | ptile [RP][kTile] | pages: page of each tile token ...
    // red [2][4][RP] after the larger of that carve-out and the epilogue's [tpar][RP][Dv] output
    // buffer.
    float* lut = smem;
    float* qp = lut + lut_floats(a, RP);
    float* ptile = qp + RP * D;
    int* pgl = reinterpret_cast<int*>(ptile + RP * kTile);  // paged with V
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
    if (W16 || p.cw > 1) {
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
    const bool pf_codes = !W16 && !PAGED && p.word_codes && nb <= 4 * kCW && !any_heavy;
    const bool pf_v = !W16 && !PAGED && HAS_V && VT != SSQ_F32 && Dv <= 8 * kVC && pv_active;  // nvc <= kVC then
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
                if (HAS_V) pgl[tid] = page;  // for the P.V loads
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
            if constexpr (W16) {
                // 16 blocks per batch: their codes are two 16-byte pieces of the token's code row,
                // loaded a batch ahead (issued after the current batch's gathers, so waiting for
                // those never waits for them) and non-temporal (the rows stream; the codebook
                // keeps the L2); the batch's codewords are gathered together, then
                // added in block order with add_block's arithmetic (FMA chain from the first
                // product), so the scores equal the block-by-block path's.  Batch slots past the
                // last block gather codeword 0 of the last block and are not used.
                constexpr int kBat = 16;
                const uint4* cr4 = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.codes) + cofs);
                uint4 cn0 = ld16g<true>(cr4), cn1 = nb > 8 ? ld16g<true>(cr4 + 1) : make_uint4(0u, 0u, 0u, 0u);
                // the block dim (2 or 4, a condition of this variant) fixed at compile time: each
                // codeword is one vector load and the FMA chain carries no per-dim branches
                auto batches = [&](auto bd_c) {
                    constexpr int BD = decltype(bd_c)::value;
                    for (int b0 = 0; b0 < nb; b0 += kBat) {
                        const uint32_t cw16[8] = {cn0.x, cn0.y, cn0.z, cn0.w, cn1.x, cn1.y, cn1.z, cn1.w};
                        uint32_t code_k[kBat];
#pragma unroll
                        for (int k = 0; k < kBat; ++k) code_k[k] = (k & 1) ? (cw16[k >> 1] >> 16) : (cw16[k >> 1] & 0xFFFFu);
                        float cv[kBat][BD];
#pragma unroll
                        for (int k = 0; k < kBat; ++k) {
                            const uint32_t cc = code_k[k] < (uint32_t)nc ? code_k[k] : (uint32_t)(nc - 1);
                            const float* c = cent + ((int64_t)min(b0 + k, nb - 1) * nc + cc) * BD;
                            if constexpr (BD == 4) {
                                const float4 v4 = *reinterpret_cast<const float4*>(c);
                                cv[k][0] = v4.x; cv[k][1] = v4.y; cv[k][2] = v4.z; cv[k][3] = v4.w;
                            } else {
                                const float2 v2 = *reinterpret_cast<const float2*>(c);
                                cv[k][0] = v2.x; cv[k][1] = v2.y;
                            }
                        }
                        if (b0 + kBat < nb) {  // the next batch's codes
                            cn0 = ld16g<true>(cr4 + ((b0 + kBat) >> 3));
                            cn1 = b0 + kBat + 8 < nb ? ld16g<true>(cr4 + ((b0 + kBat) >> 3) + 1) : make_uint4(0u, 0u, 0u, 0u);
                        }
#pragma unroll
                        for (int k = 0; k < kBat; ++k) {
                            const int blk = b0 + k;
                            if (blk >= nb) break;
                            if (ssq_is_heavy(a.heavy_mask[0], a.heavy_mask[1], blk)) {
                                add_block(blk, code_k[k]);
                                continue;
                            }
                            float e_acc[RP];
#pragma unroll
                            for (int r = 0; r < RP; ++r) e_acc[r] = qp[r * D + blk * BD] * cv[k][0];
#pragma unroll
                            for (int d = 1; d < BD; ++d)
#pragma unroll
                                for (int r = 0; r < RP; ++r) e_acc[r] = fmaf(qp[r * D + blk * BD + d], cv[k][d], e_acc[r]);
#pragma unroll
                            for (int r = 0; r < RP; ++r) s[r] += e_acc[r];
                        }
                    }
                };
                if (bd == 4) batches(std::integral_constant<int, 4>{});
                else batches(std::integral_constant<int, 2>{});
            } else if (p.cw > 1 && bd <= 4) {
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
                // kVB token rows per batch, every load of a batch issued before the arithmetic
                // (row indexes clamped to the tile's last token; the clamped slots are skipped).
                // One row at a time in the other variants: they also hold the prefetch path, whose
                // registers a batch would add to (measured slower at configs 3 and 5).
                constexpr int kVB = !W16 ? 1 : VT == SSQ_F32 ? 4 : 8;
                const int64_t vbase = (int64_t)b * a.v_sb + (int64_t)kv * a.v_sh + pv_d * 8;
                for (int tt0 = pv_t; tt0 < nt; tt0 += kVB * tpar) {
                    VRaw8<VT> raw[kVB];
#pragma unroll
                    for (int k = 0; k < kVB; ++k)
                        raw[k] = load_v8_raw<VT, W16>(a.v, vbase + (int64_t)(t0 + min(tt0 + k * tpar, nt - 1)) * a.v_st);
#pragma unroll
                    for (int k = 0; k < kVB; ++k) {
                        const int tt = tt0 + k * tpar;
                        if (tt >= nt) break;
                        float v[8];
                        unpack_v8<VT>(raw[k], v);
#pragma unroll
                        for (int r = 0; r < RP; ++r) {
                            const float pr = ptile[r * kTile + tt];
#pragma unroll
                            for (int j = 0; j < 8; ++j) acc[r][j] = fmaf(pr, v[j], acc[r][j]);
                        }
                    }
                }
            } else {
                // V pages [P, Hkv, Dv, page]: 8 consecutive tokens of one dim per load, kVB chunks
                // per batch with every load issued before the arithmetic; each chunk's page is the
                // one its first token's score read (pgl: no block-table load in the chain).  Chunk
                // indexes are clamped to the tile's last chunk; the clamped slots are skipped.
                constexpr int kVB = VT == SSQ_F32 ? 4 : 8;
                const int nchunks = (nt + 7) >> 3;
                const int64_t vhead = (int64_t)kv * a.v_sh + (int64_t)pv_d * a.v_st;
                for (int c0 = pv_t; c0 < nchunks; c0 += kVB * tpar) {
                    VRaw8<VT> raw[kVB];
#pragma unroll
                    for (int k = 0; k < kVB; ++k) {
                        const int tt = min(c0 + k * tpar, nchunks - 1) * 8;
                        const int t = t0 + tt;
                        const int off = t - (t / a.page_size) * a.page_size;
                        raw[k] = load_v8_raw<VT, W16>(a.v, (int64_t)pgl[tt] * a.v_sb + vhead + off);
                    }
#pragma unroll
                    for (int k = 0; k < kVB; ++k) {
                        const int ch = c0 + k * tpar;
                        if (ch >= nchunks) break;
                        const int tt = ch * 8;
                        float v[8];
                        unpack_v8<VT>(raw[k], v);
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

template <int RP, bool PAGED, bool HAS_V, int VT, bool W16>
int launch_t(const DecodeParams& dp, const SsqGenericLaunch& gl, hipStream_t st) {
    auto kern = k_decode_generic<RP, PAGED, HAS_V, VT, W16>;
    int rc = ssq_allow_lds((const void*)kern, (int)kMaxSmem, "hipFuncSetAttribute(decode)");
    if (rc) return rc;
    dim3 grid(gl.n_splits, gl.n_groups, dp.a.batch * dp.a.num_kv_heads);
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), gl.smem, st, dp);
    return ssq_check_hip(hipGetLastError(), "k_decode_generic launch");
}

template <int RP, bool PAGED, bool HAS_V, bool W16>
int launch_vt(const DecodeParams& dp, const SsqGenericLaunch& gl, hipStream_t st) {
    if (!HAS_V) return launch_t<RP, PAGED, HAS_V, SSQ_BF16, W16>(dp, gl, st);
    switch (dp.a.v_dtype) {
        case SSQ_BF16: return launch_t<RP, PAGED, HAS_V, SSQ_BF16, W16>(dp, gl, st);
        case SSQ_F16: return launch_t<RP, PAGED, HAS_V, SSQ_F16, W16>(dp, gl, st);
        default: return launch_t<RP, PAGED, HAS_V, SSQ_F32, W16>(dp, gl, st);
    }
}

template <int RP, bool W16>
int launch_rp(const DecodeParams& dp, const SsqGenericLaunch& gl, hipStream_t st) {
    if (dp.a.layout == SSQ_PAGED)
        return gl.has_v ? launch_vt<RP, true, true, W16>(dp, gl, st) : launch_vt<RP, true, false, W16>(dp, gl, st);
    return gl.has_v ? launch_vt<RP, false, true, W16>(dp, gl, st) : launch_vt<RP, false, false, W16>(dp, gl, st);
}

template <bool W16>
int launch_generic(const DecodeParams& dp, const SsqGenericLaunch& gl, hipStream_t st) {
    switch (gl.RP) {
        case 1: return launch_rp<1, W16>(dp, gl, st);
        case 2: return launch_rp<2, W16>(dp, gl, st);
        case 4: return launch_rp<4, W16>(dp, gl, st);
        default: return launch_rp<8, W16>(dp, gl, st);
    }
}

}  // namespace

// the 16-bit-code variants (ssq_decode_generic_w16.hip)
int ssq_generic_w16(const SsqGenericParams& dp, const SsqGenericLaunch& gl, hipStream_t st);

// the staged-codebook kernel for 16-bit codes over long contexts (ssq_decode_wide.hip): its LDS
// bytes at RP rows per workgroup, whether the codebook and values suit it, and its launch
size_t ssq_decode_wide_smem(const ssq_decode_args& a, int RP);
bool ssq_decode_wide_fits(const ssq_decode_args& a);
int ssq_decode_wide(const SsqGenericParams& dp, int RP, int n_groups, size_t smem, hipStream_t st);
