// Fused VQ-key decode over vLLM-style pages with P.V on the matrix cores (gfx950): the kernel
// template and its launchers.  The host plan is in ssq_decode_mfma.hip; the instantiations are
// spread over ssq_decode_mfma_lut*.hip (compiled in parallel).
//
// Same mathematics as the generic kernel (ssq_decode.hip): LUT scores
// (triton_kernels.py:381-408, :174-196), online softmax, probabilities cast to
// the value dtype before P.V (vllm_attn_backend.py:251-252).  Different mapping:
//
//   workgroup = 4 waves (one per SIMD) for one (batch, KV head, context split); LUT [nb][nc][RP]
//   fp32 in LDS (<= ~144 KiB, so one workgroup per CU).
//   wave      = streams 64-token tiles (4 pages of 16) independently with its own
//               running (max, sum, O); waves merge through LDS at the end.
//   scores    = one token per lane: nb ds_read_b128 LUT gathers give all RP rows.
//   P.V       = v_mfma_f32_16x16x32_bf16 (or _f16): A = P [16 rows x 32 tokens]
//               staged through a per-wave LDS strip; B = V [32 tokens x 16 dims]
//               read straight from the page: vLLM's value page is dim-major
//               ([Dv][page]), so the 8 consecutive tokens of one dim that a lane
//               supplies to the B operand are one 16-byte load.
//
// The same kernel with CT = true reads contiguous rows (codes [B, Hkv, T, nb], V [B, Hkv, T, 128],
// token-major) for head dims past the contiguous MFMA kernel's 64: V tiles load as coalesced
// 256-byte rows and pass through a per-wave LDS buffer 16 tokens at a time, read back transposed
// (ds_read_b64_tr_b16) as B operands of v_mfma_f32_16x16x16.
#pragma once

#include "ssq_decode_paged.h"

#include <math.h>

#include <type_traits>

// launch plan of the paged LUT kernel (and of the 4x4-MFMA-scores kernel it hands shapes to)
struct SsqMfmaPlan {
    int RP, DT, split_len, n_splits;
    int rg, n_groups;  // query rows per row group, row groups
    bool q4;           // k_decode_paged_q4 (4x4-MFMA scores) in place of the LUT kernel
    bool ct;           // contiguous rows (the LUT kernel with CT = true)
    size_t smem, ws_bytes;
};

namespace {

// LUT codewords per block: 256, or 64 for 64-codeword codebooks (a table a quarter the size)
__host__ __device__ inline int lut_nc(const ssq_decode_args& a) { return a.n_centroids == 64 ? 64 : kNC; }
// LDS carve-up (floats): lut [nb*nc*RP] | qp [RP*D] | pstrip [waves][RP][64] (16-bit) | then either
// pages [split_len/16] (int32) or, for contiguous rows, vbuf [waves][16][kVRow] (16-bit)
constexpr int kVRow = 128 + 16;  // vbuf row: 128 dims and 16 of padding (the transposed reads' banks)
__host__ __device__ inline size_t lut_floats(const ssq_decode_args& a, int RP) {
    return (size_t)a.n_blocks * lut_nc(a) * RP;
}
__host__ __device__ inline size_t pstrip_offset(const ssq_decode_args& a, int RP) {
    return (lut_floats(a, RP) + (size_t)RP * a.head_dim + 3) & ~(size_t)3;
}
__host__ __device__ inline size_t pages_offset(const ssq_decode_args& a, int RP) {
    return pstrip_offset(a, RP) + (size_t)kWaves * RP * kTileTok / 2;
}
inline size_t mfma_smem(const ssq_decode_args& a, int RP, int split_len, bool ct = false) {
    const size_t main = pages_offset(a, RP) + (ct ? (size_t)kWaves * 16 * kVRow / 2 : (size_t)split_len / kPage);
    const size_t merge = (size_t)kWaves * RP * (a.value_dim + 2);
    return (main > merge ? main : merge) * sizeof(float);
}

// Contiguous rows (codes [B, Hkv, T, nb] bytes, V [B, Hkv, T, 128]): cb0 and vb0 (bytes) point at the
// split's first token of this (batch, KV head).  A lane loads its token's code row; the values arrive
// as four 16-token chunks, chunk c in the flat registers 4c .. 4c + 3 of R.v, register 4c + i holding
// dims 8 (lane % 16) .. + 7 of token 16c + 4i + lane / 16 (16 lanes read one 256-byte row).  Tokens
// past the split's end read its last token: finite values, given probability 0.  Offsets from the
// tile's first token are 32-bit (the plan keeps 64 tokens' strides below 2^31 bytes).
// A contiguous tile's registers: the paged tile's, and with a mask (MK) the additive mask of each row
// for this lane's token (rows past the workgroup's last one re-read that row's entry).
template <int NB, int DT, int RP, bool MK, bool HV>
struct TileRegsCT : TileRegs<NB, DT, 0> {
    float mk[MK ? RP : 1];
    uint32_t pt[HV ? 16 : 1];  // passthrough values (raw bits) of this lane's token
};

template <int NB, int DT, int RP, bool MK, bool NV, bool HV>
__device__ __forceinline__ void issue_tile_ct(const MfmaParams& p, int b, int kv, int t_begin, int t_end, int tile,
                                              int lane, const uint8_t* cb0, const uint8_t* vb0,
                                              TileRegsCT<NB, DT, RP, MK, HV>& R) {
    static_assert(DT == 8, "contiguous LUT tiles carry 128-dim values");
    const ssq_decode_args& a = p.a;
    const int rel = tile * kTileTok;
    const int lim = t_end - 1 - t_begin - rel;  // the split's last token, from the tile's first (>= 0)
    const uint8_t* ctile = cb0 + (int64_t)rel * a.c_st;
    const uint8_t* vtile = vb0 + (int64_t)rel * 2 * a.v_st;
    const uint32_t coff = (uint32_t)min(lane, lim) * (uint32_t)a.c_st;
    if constexpr (NB >= 16) {
#pragma unroll
        for (int i = 0; i < NB / 16; ++i) R.c[i] = *reinterpret_cast<const uint4*>(ctile + coff + 16 * i);
    } else {
        R.c8 = *reinterpret_cast<const uint2*>(ctile + coff);
    }
    if constexpr (!NV) {
        const uint32_t vst = 2u * (uint32_t)a.v_st, dcol = 16u * (uint32_t)(lane & 15);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const uint32_t tok = (uint32_t)min(16 * (k >> 2) + 4 * (k & 3) + (lane >> 4), lim);
            const uint32_t off = tok * vst + dcol;  // one 32-bit offset: the uniform-base load form
            R.v[k >> 3][k & 7] = load_stream(reinterpret_cast<const uint16_t*>(vtile + off));
        }
    }
    if constexpr (MK) {
        const int row0 = blockIdx.z * p.rg, nr = min(p.rg, p.rows - row0);
        const int64_t t = t_begin + rel + min(lane, lim);
#pragma unroll
        for (int r = 0; r < RP; ++r) {
            const int rr = row0 + min(r, nr - 1);
            const int g = rr / a.q_len, qi = rr - g * a.q_len;
            const int h = kv * p.G + g;
            R.mk[r] = a.mask[(int64_t)b * a.m_sb + (int64_t)h * a.m_sh + (int64_t)qi * a.m_sl + t * a.m_st];
        }
    }
    if constexpr (HV) {  // n_hd (8 or 16) consecutive 16-bit values: two 16-byte loads (the second
                         // re-reads the first with 8), straight-line like the tile's other loads
        const int64_t row = (int64_t)b * a.pt_sb + (int64_t)kv * a.pt_sh + (int64_t)(t_begin + rel + min(lane, lim)) * a.pt_st;
        const uint4* src = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.pt) + row + p.hoff[0]);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint4 w = src[min(j, p.n_hd / 8 - 1)];
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                R.pt[8 * j + 2 * k] = ww[k] & 0xFFFFu;
                R.pt[8 * j + 2 * k + 1] = ww[k] >> 16;
            }
        }
    }
}

// the wave's LDS writes before this point are seen by its reads after it (an ordering point for the
// compiler: one wave's LDS operations execute in order)
__device__ __forceinline__ void lds_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ v4f mfma16_bf16(const uint2& a, const uint2& b, v4f c) {
    typedef short v4s_t __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(v4s_t, a), __builtin_bit_cast(v4s_t, b), c, 0,
                                                     0, 0);
}
__device__ __forceinline__ v4f mfma16_f16(const uint2& a, const uint2& b, v4f c) {
    typedef _Float16 v4h_t __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4h_t, a), __builtin_bit_cast(v4h_t, b), c, 0, 0,
                                                 0);
}

// P.V over a contiguous tile (after tile_probs): per 16-token chunk, the chunk's values go row-major
// into the wave's LDS buffer [16][kVRow] and come back transposed with ds_read_b64_tr_b16 (within
// each 16-lane group g = lane / 16, lane l reads 4 elements of row 4g + l / 4 and receives dim
// 16 dt + l of rows 4g .. 4g + 3): the B operand of v_mfma_f32_16x16x16, tokens 4g .. 4g + 3 of one
// dim.  A = P [16 rows x 16 tokens] from the strip.  The 16-element row padding puts a group's four
// rows on distinct LDS banks.
template <int RP, int DT, int VT, int NB>
__device__ __forceinline__ void tile_pv_ct(const uint16_t* pstrip, uint16_t* vbuf, int lane,
                                           const TileRegs<NB, DT, 0>& R, v4f (&acc)[DT]) {
    typedef short v4s_t __attribute__((ext_vector_type(4)));
    const int l16 = lane & 15, lg = lane >> 4;
    const uint16_t* src = vbuf + (4 * lg + (l16 >> 2)) * kVRow + 4 * (l16 & 3);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = 4 * c + i;
            *reinterpret_cast<uint4*>(vbuf + (4 * i + lg) * kVRow + 8 * l16) = R.v[k >> 3][k & 7];
        }
        lds_wave_sync();
        uint2 af = make_uint2(0, 0);
        if (l16 < RP) af = *reinterpret_cast<const uint2*>(pstrip + l16 * kTileTok + 16 * c + 4 * lg);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const v4s_t bv = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) v4s_t*)(src + 16 * dt));
            const uint2 b2 = __builtin_bit_cast(uint2, bv);
            acc[dt] = VT == SSQ_BF16 ? mfma16_bf16(af, b2, acc[dt]) : mfma16_f16(af, b2, acc[dt]);
        }
        lds_wave_sync();  // the chunk's transposed reads are done before the next chunk's writes
    }
}

// one tile's loads: contiguous rows (CT, with the mask when MK, codes only when NV) or pages
template <bool CT, bool MK, bool NV, bool HV, int RP, int NB, int DT, int PB, class TR>
__device__ __forceinline__ void issue_any(const MfmaParams& p, int b, int kv, const int* pages, int t_begin, int t_end,
                                          int tile, int lane, const uint8_t* cbase, const uint16_t* vbase,
                                          const uint8_t* cb0, const uint8_t* vb0, TR& R) {
    if constexpr (CT) {
        issue_tile_ct<NB, DT, RP, MK, NV, HV>(p, b, kv, t_begin, t_end, tile, lane, cb0, vb0, R);
    } else {
        issue_tile<NB, DT, PB>(p.a, pages, t_begin, t_end, tile, lane, cbase, vbase, R);
    }
}

template <int RP, int DT, int VT, int NB, int NC, int PB, bool CT, bool MK, bool NV, bool HV, class TR>
__device__ __forceinline__ void compute_tile(const MfmaParams& p, const float* lut, const float (&qh)[HV ? RP : 1][16],
                                             uint16_t* pstrip, uint16_t* vbuf,
                                             int b, int kv, int t_begin, int t_end, int tile, int lane, TR& R,
                                             float (&m_run)[RP], float (&l_lane)[RP], v4f (&acc)[DT]) {
    const int t0 = t_begin + tile * kTileTok;
    float s[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) s[r] = 0.f;
    {
        // LUT gathers a batch of KB blocks at a time: all KB reads are issued before the first
        // is consumed (one wave per SIMD hides no LDS latency otherwise); the sums still run in
        // block order from 0.  Lanes past the end gather too (their codes are a valid token's)
        // and are dropped by tile_softmax_pv.
        constexpr int KB = RP >= 8 ? 4 : 8;
        constexpr int NVEC = RP >= 4 ? RP / 4 : 1;  // float4 (or one float2 / float) per block
#pragma unroll
        for (int b0 = 0; b0 < NB; b0 += KB) {
            float4 ev[KB][NVEC];
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                const int blk = b0 + k;
                uint32_t code;
                if constexpr (PB > 0) {  // PB-bit codes, 32 / PB to a word, low bits first
                    constexpr int kVpe = 32 / PB;
                    code = (R.pk[blk / kVpe] >> ((blk % kVpe) * PB)) & ((1u << PB) - 1u);
                } else {
                    const int wi = blk >> 2;
                    uint32_t word;
                    if (NB >= 16) {
                        const uint4 c = R.c[wi >> 2];
                        word = (wi & 3) == 0 ? c.x : (wi & 3) == 1 ? c.y : (wi & 3) == 2 ? c.z : c.w;
                    } else {
                        word = (wi & 1) ? R.c8.y : R.c8.x;
                    }
                    code = (word >> (8 * (blk & 3))) & 0xFFu;
                }
                if constexpr (NC < 256) code = min(code, (uint32_t)(NC - 1));  // codes past the codebook
                const float* e = lut + ((size_t)blk * NC + code) * RP;
                if (RP >= 4) {
#pragma unroll
                    for (int j = 0; j < NVEC; ++j) ev[k][j] = *reinterpret_cast<const float4*>(e + 4 * j);
                } else if (RP == 2) {
                    const float2 v = *reinterpret_cast<const float2*>(e);
                    ev[k][0] = make_float4(v.x, v.y, 0.f, 0.f);
                } else {
                    ev[k][0] = make_float4(e[0], 0.f, 0.f, 0.f);
                }
            }
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                if (RP >= 4) {
#pragma unroll
                    for (int j = 0; j < NVEC; ++j) {
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
    if constexpr (NV) {  // scores only
        tile_store_scores<RP>(p, b, kv, t0, t_end, lane, s);
    } else if constexpr (CT) {
        if constexpr (HV) {  // passthrough dims: q_perm . stored value, after the LUT sums
            const ssq_decode_args& a = p.a;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (i < p.n_hd) {  // wave-uniform
                    const float x = ssq_bits_to_f32(R.pt[i], a.pt_dtype);
#pragma unroll
                    for (int r = 0; r < RP; ++r) s[r] = fmaf(qh[r][i], x, s[r]);
                }
            }
        }
        if constexpr (MK) {
            const int nr = min(p.rg, p.rows - (int)blockIdx.z * p.rg);
#pragma unroll
            for (int r = 0; r < RP; ++r) s[r] += r < nr ? R.mk[r] : 0.f;
        }
        tile_probs<RP, DT, VT>(p, pstrip, b, kv, t0, t_end, lane, s, m_run, l_lane, acc);
        tile_pv_ct<RP, DT, VT, NB>(pstrip, vbuf, lane, R, acc);
    } else {
        tile_softmax_pv<RP, DT, VT, NB, PB>(p, pstrip, b, kv, t0, t_end, lane, s, R, m_run, l_lane, acc);
    }
}

// vector of N floats from memory (N = 1, 2, 4 or a multiple of 4; 4N-byte aligned)
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

// LUT[e][r] = sum_d qp[r][blk*BD + d] * C[e][d] for this thread's entries e = tid + k*kThreads
// (blk = e / NC): FMA chain over d from the first product (triton_kernels.py:381-408).  A batch
// of entries loads its codewords and query sub-vectors as vectors before any arithmetic, so the
// build costs a few memory / LDS latencies instead of one per element.
template <int RP, int NB, int BD, int NC>
__device__ __forceinline__ void build_lut(const float* __restrict__ cent, const float* __restrict__ qp,
                                          float* __restrict__ lut, int D, int tid) {
    constexpr int kPer = NB * NC / kThreads;
    constexpr int kB = kPer < 128 / BD ? kPer : 128 / BD;  // up to 128 codeword floats in flight
#pragma unroll
    for (int k0 = 0; k0 < kPer; k0 += kB) {
        float c[kB][BD];
#pragma unroll
        for (int kk = 0; kk < kB; ++kk) {
            if (k0 + kk < kPer) load_vec<BD>(cent + (int64_t)(tid + (k0 + kk) * kThreads) * BD, c[kk]);
        }
#pragma unroll
        for (int kk = 0; kk < kB; ++kk) {
            if (k0 + kk >= kPer) break;
            const int e = tid + (k0 + kk) * kThreads;
            const float* qb = qp + (e / NC) * BD;
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

// any block_dim: one element at a time
template <int RP, int NB, int NC>
__device__ void build_lut_any(const float* __restrict__ cent, const float* __restrict__ qp, float* __restrict__ lut,
                              int D, int bd, int tid) {
    for (int e = tid; e < NB * NC; e += kThreads) {
        const float* c = cent + (int64_t)e * bd;
        const float* qb = qp + (e / NC) * bd;
        float acc[RP];
#pragma unroll
        for (int r = 0; r < RP; ++r) acc[r] = qb[r * D] * c[0];
        for (int d = 1; d < bd; ++d) {
            const float cd = c[d];
#pragma unroll
            for (int r = 0; r < RP; ++r) acc[r] = fmaf(qb[r * D + d], cd, acc[r]);
        }
#pragma unroll
        for (int r = 0; r < RP; ++r) lut[(size_t)e * RP + r] = acc[r];
    }
}

// NC: LUT codewords per block (256, or 64); PB: packed code bits (0 = byte codes); CT: contiguous rows,
// MK: with an additive mask, NV: scores only, HV: passthrough blocks (all on contiguous rows only)
template <int RP, int DT, int VT, int NB, int NC, int PB, bool CT, bool MK, bool NV, bool HV>
__global__ __launch_bounds__(kThreads) void k_decode_mfma(const MfmaParams p) {
    extern __shared__ __align__(16) float smem[];
    const ssq_decode_args& a = p.a;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar loop control
    const int bk = blockIdx.x;
    const int split = blockIdx.y;
    const int b = bk / a.num_kv_heads;
    const int kv = bk - b * a.num_kv_heads;
    const int D = a.head_dim, bd = a.block_dim;
    const int row0 = blockIdx.z * p.rg;          // this workgroup's query rows: row0 .. row0 + nr - 1
    const int nr = min(p.rg, p.rows - row0);     // <= RP
    const int T = CT ? a.seq_len : min(a.seq_lens[b], a.seq_len);
    const int t_begin = split * p.split_len;
    const int t_end = min(T, t_begin + p.split_len);

    float* lut = smem;
    float* qp = smem + lut_floats(a, RP);
    uint16_t* pstrip = reinterpret_cast<uint16_t*>(smem + pstrip_offset(a, RP)) + wave * RP * kTileTok;
    int* pages = reinterpret_cast<int*>(smem + pages_offset(a, RP));
    uint16_t* vbuf = reinterpret_cast<uint16_t*>(smem + pages_offset(a, RP)) + wave * 16 * kVRow;  // CT

    // ---- prologue.  The query rows are loaded unpermuted (coalesced, independent of the
    // permutation) together with this thread's permutation entries and the first block-table
    // pass: one memory latency.  The rows are scaled into the LUT region (free until the LUT is
    // built), then permuted LDS-to-LDS into qp.
    const int32_t* btab = CT ? nullptr : a.block_table + (int64_t)b * a.bt_sb + t_begin / kPage;
    const int n_pages = !CT && t_end > t_begin ? (t_end - t_begin + kPage - 1) / kPage : 0;
    const float* cent = a.cent + (int64_t)kv * a.cent_sh;
    const int64_t* perm = a.perm + (int64_t)kv * a.perm_sh;
    constexpr int kQP = (RP * 256 + kThreads - 1) / kThreads;  // head_dim <= 256 on this kernel
    constexpr int kBT = 8;                                      // block-table entries per thread per pass
    float qv[kQP];
    bool ok[kQP];
    int64_t pv[kQP];
    {
        int64_t src[kQP];
#pragma unroll
        for (int k = 0; k < kQP; ++k) {
            const int e = tid + k * kThreads;
            const int r = e / D, j = e - r * D;
            pv[k] = perm[e < RP * D ? j : 0];
            ok[k] = e < RP * D && r < nr;
            src[k] = 0;  // rows past nr read element 0 and are zeroed
            if (ok[k]) {
                const int g = (row0 + r) / a.q_len, qi = row0 + r - g * a.q_len;
                const int h = kv * p.G + g;
                src[k] = (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)qi * a.q_sl + j;
            }
        }
        int ent[kBT];
#pragma unroll
        for (int k = 0; k < kBT; ++k) {
            const int i = k * kThreads + tid;
            ent[k] = i < n_pages ? btab[i] : 0;
        }
        ssq_load_elems(a.q, a.q_dtype, src, qv);
#pragma unroll
        for (int k = 0; k < kBT; ++k) {
            const int i = k * kThreads + tid;
            if (i < n_pages) pages[i] = ent[k];
        }
    }
    for (int base = kBT * kThreads; base < n_pages; base += kBT * kThreads) {  // longer splits
        int ent[kBT];
#pragma unroll
        for (int k = 0; k < kBT; ++k) {
            const int i = base + k * kThreads + tid;
            ent[k] = i < n_pages ? btab[i] : 0;
        }
#pragma unroll
        for (int k = 0; k < kBT; ++k) {
            const int i = base + k * kThreads + tid;
            if (i < n_pages) pages[i] = ent[k];
        }
    }
    float* qraw = lut;  // [RP][D], scaled
#pragma unroll
    for (int k = 0; k < kQP; ++k) {
        const int e = tid + k * kThreads;
        if (e < RP * D) qraw[e] = !ok[k] ? 0.f : a.has_scale ? ssq_round_to(qv[k] * a.scale, a.q_dtype) : qv[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kQP; ++k) {
        const int e = tid + k * kThreads;
        const int r = e / D;
        if (e < RP * D) qp[e] = qraw[r * D + (int)min((uint64_t)pv[k], (uint64_t)(D - 1))];
    }
    __syncthreads();
    // the first tile's codes and values are independent of the LUT: put them in flight before building it
    const uint16_t* vbase = reinterpret_cast<const uint16_t*>(a.v) + (int64_t)kv * a.v_sh + (int64_t)(lane & 15) * a.v_st;
    const uint8_t* cbase = PB > 0 ? reinterpret_cast<const uint8_t*>(reinterpret_cast<const uint32_t*>(a.codes) +
                                                                     (int64_t)kv * a.c_sh)
                                  : a.codes + (int64_t)kv * a.c_sh;
    const uint8_t* cb0 = a.codes + (int64_t)b * a.c_sb + (int64_t)kv * a.c_sh + (int64_t)t_begin * a.c_st;  // CT
    const uint8_t* vb0 = reinterpret_cast<const uint8_t*>(a.v) +
                         2 * ((int64_t)b * a.v_sb + (int64_t)kv * a.v_sh + (int64_t)t_begin * a.v_st);  // CT
    const int n_tiles = (t_end - t_begin + kTileTok - 1) / kTileTok;
    static_assert(CT || (!MK && !NV && !HV), "masks, scores only and passthrough are contiguous-path variants");
    using Regs = std::conditional_t<CT, TileRegsCT<NB, DT, RP, MK, HV>, TileRegs<NB, DT, PB>>;
    Regs RA, RB;
    int tile = wave;
    // Tile loads are issued unconditionally (a wave past the last tile re-reads tile n_tiles-1,
    // mostly from L2): every path then carries the same queue of outstanding loads, so the
    // compiler's vmcnt waits for the tile being computed never drain the tile behind it.
    const int last_tile = n_tiles > 0 ? n_tiles - 1 : 0;
    if (n_tiles > 0)
        issue_any<CT, MK, NV, HV, RP, NB, DT, PB>(p, b, kv, pages, t_begin, t_end, min(tile, last_tile), lane, cbase,
                                              vbase, cb0, vb0, RA);
    switch (bd) {
        case 1: build_lut<RP, NB, 1, NC>(cent, qp, lut, D, tid); break;
        case 2: build_lut<RP, NB, 2, NC>(cent, qp, lut, D, tid); break;
        case 4: build_lut<RP, NB, 4, NC>(cent, qp, lut, D, tid); break;
        case 8: build_lut<RP, NB, 8, NC>(cent, qp, lut, D, tid); break;
        default: build_lut_any<RP, NB, NC>(cent, qp, lut, D, bd, tid); break;
    }
    if constexpr (HV) {  // passthrough blocks score from their stored values: zero their LUT rows
        __syncthreads();
        for (int e = tid; e < NB * NC * RP; e += kThreads)
            if ((a.heavy_mask[0] >> (e / (NC * RP))) & 1ull) lut[e] = 0.f;
    }
    __syncthreads();
    // the permuted query rows at the passthrough dims, in registers for the whole stream
    float qh[HV ? RP : 1][16];
#pragma unroll
    for (int r = 0; r < (HV ? RP : 1); ++r) {
#pragma unroll
        for (int i = 0; i < 16; ++i) qh[r][i] = HV && i < p.n_hd ? qp[r * D + p.hdim[i]] : 0.f;
    }

    // ---- stream tiles, two in flight per wave (A/B register sets, no copies)
    float m_run[RP], l_lane[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) { m_run[r] = -INFINITY; l_lane[r] = 0.f; }
    v4f acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = (v4f){0.f, 0.f, 0.f, 0.f};
    if constexpr (DT > 8) {
        // 256-dim values: two tiles' V fragments would take all 256 registers, so one register
        // set; a wave issues its next tile once this one is consumed (the other waves' loads keep
        // the memory busy meanwhile)
        while (tile < n_tiles) {
            compute_tile<RP, DT, VT, NB, NC, PB, CT, MK, NV, HV>(p, lut, qh, pstrip, vbuf, b, kv, t_begin, t_end, tile, lane,
                                                             RA, m_run, l_lane, acc);
            tile += kWaves;
            if (tile >= n_tiles) break;
            issue_any<CT, MK, NV, HV, RP, NB, DT, PB>(p, b, kv, pages, t_begin, t_end, tile, lane, cbase, vbase, cb0, vb0,
                                                  RA);
        }
    } else {
        while (tile < n_tiles) {
            issue_any<CT, MK, NV, HV, RP, NB, DT, PB>(p, b, kv, pages, t_begin, t_end, min(tile + kWaves, last_tile), lane,
                                                  cbase, vbase, cb0, vb0, RB);
            compute_tile<RP, DT, VT, NB, NC, PB, CT, MK, NV, HV>(p, lut, qh, pstrip, vbuf, b, kv, t_begin, t_end, tile, lane,
                                                             RA, m_run, l_lane, acc);
            tile += kWaves;
            if (tile >= n_tiles) break;
            issue_any<CT, MK, NV, HV, RP, NB, DT, PB>(p, b, kv, pages, t_begin, t_end, min(tile + kWaves, last_tile), lane,
                                                  cbase, vbase, cb0, vb0, RA);
            compute_tile<RP, DT, VT, NB, NC, PB, CT, MK, NV, HV>(p, lut, qh, pstrip, vbuf, b, kv, t_begin, t_end, tile, lane,
                                                             RB, m_run, l_lane, acc);
            tile += kWaves;
        }
    }

    if constexpr (NV) return;  // scores only: every tile's scores are stored

    // ---- merge the waves' (m, l, O) through LDS (the LUT is no longer needed)
    float l_w[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) l_w[r] = wave_sum(l_lane[r]);
    __syncthreads();
    float* mbuf = smem;                         // [waves][RP]
    float* lbuf = mbuf + kWaves * RP;           // [waves][RP]
    float* obuf = lbuf + kWaves * RP;           // [waves][RP][Dv]
    const int Dv = DT * 16;
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RP; ++r) { mbuf[wave * RP + r] = m_run[r]; lbuf[wave * RP + r] = l_w[r]; }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 4 * (lane >> 4) + i;
        if (row < RP) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) obuf[((size_t)wave * RP + row) * Dv + 16 * dt + (lane & 15)] = acc[dt][i];
        }
    }
    __syncthreads();
    const int n_rows_all = a.batch * a.num_q_heads * a.q_len;
    for (int e = tid; e < nr * Dv; e += kThreads) {
        const int r = e / Dv, dv = e - r * Dv;
        float M = -INFINITY;
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, mbuf[w * RP + r]);
        float L = 0.f, o = 0.f;
        for (int w = 0; w < kWaves; ++w) {
            const float mw = mbuf[w * RP + r];
            if (mw == -INFINITY) continue;
            const float f = __expf(mw - M);
            L += lbuf[w * RP + r] * f;
            o += obuf[((size_t)w * RP + r) * Dv + dv] * f;
        }
        const int g = (row0 + r) / a.q_len, qi = row0 + r - g * a.q_len;
        const int h = kv * p.G + g;
        const int rid = (b * a.num_q_heads + h) * a.q_len + qi;
        if (p.n_splits == 1) {
            ssq_store_elem(a.out, a.v_dtype, (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)qi * a.o_sl + dv, o / L);
            if (a.lse && dv == 0) a.lse[rid] = M + logf(L);
        } else {
            p.ws_o[((size_t)split * n_rows_all + rid) * Dv + dv] = o;
            if (dv == 0) {
                p.ws_m[(size_t)split * n_rows_all + rid] = M;
                p.ws_l[(size_t)split * n_rows_all + rid] = L;
            }
        }
    }
}

template <int RP, int DT, int VT, int NB, int NC = kNC, int PB = 0, bool CT = false, bool MK = false,
          bool NV = false, bool HV = false>
int launch(const MfmaParams& mp, const SsqMfmaPlan& pl, hipStream_t st) {
    auto kern = k_decode_mfma<RP, DT, VT, NB, NC, PB, CT, MK, NV, HV>;
    int rc = ssq_allow_lds((const void*)kern, (int)kMaxSmem, "hipFuncSetAttribute(decode_mfma)");
    if (rc) return rc;
    dim3 grid(mp.a.batch * mp.a.num_kv_heads, pl.n_splits, pl.n_groups);
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), pl.smem, st, mp);
    return ssq_check_hip(hipGetLastError(), "k_decode_mfma launch");
}

template <int RP, int DT, int VT>
int launch_nb(const MfmaParams& mp, const SsqMfmaPlan& pl, hipStream_t st) {
    switch (mp.a.n_blocks) {
        case 8: return launch<RP, DT, VT, 8>(mp, pl, st);
        case 16: if constexpr (RP <= 8) return launch<RP, DT, VT, 16>(mp, pl, st); break;
        case 32: if constexpr (RP <= 4) return launch<RP, DT, VT, 32>(mp, pl, st); break;
        default: if constexpr (RP <= 2) return launch<RP, DT, VT, 64>(mp, pl, st); break;
    }
    return ssq_fail(SSQ_ERR_UNSUPPORTED, "MFMA decode: LUT of %d rows x %d blocks exceeds LDS", RP, mp.a.n_blocks);
}

template <int RP, int VT>
int launch_dt(const MfmaParams& mp, const SsqMfmaPlan& pl, hipStream_t st) {
    switch (pl.DT) {
        case 4: return launch_nb<RP, 4, VT>(mp, pl, st);
        case 8: return launch_nb<RP, 8, VT>(mp, pl, st);
        default: return launch_nb<RP, 16, VT>(mp, pl, st);
    }
}

template <int RP>
int launch_vt(const MfmaParams& mp, const SsqMfmaPlan& pl, hipStream_t st) {
    return mp.a.v_dtype == SSQ_BF16 ? launch_dt<RP, SSQ_BF16>(mp, pl, st) : launch_dt<RP, SSQ_F16>(mp, pl, st);
}

// 64-codeword LUT kernel (lut64_shape): bf16 V, byte or 6-bit codes
template <int RP, int DT, int PB>
int lut64_nb(const MfmaParams& mp, const SsqMfmaPlan& pl, hipStream_t st) {
    switch (mp.a.n_blocks) {
        case 16: return launch<RP, DT, SSQ_BF16, 16, 64, PB>(mp, pl, st);
        case 32: return launch<RP, DT, SSQ_BF16, 32, 64, PB>(mp, pl, st);
        default: return launch<RP, DT, SSQ_BF16, 64, 64, PB>(mp, pl, st);
    }
}
template <int PB>
int lut64_rp(const MfmaParams& mp, const SsqMfmaPlan& pl, hipStream_t st) {
    switch (pl.RP) {
        case 2: return pl.DT == 4 ? lut64_nb<2, 4, PB>(mp, pl, st) : lut64_nb<2, 8, PB>(mp, pl, st);
        case 4: return pl.DT == 4 ? lut64_nb<4, 4, PB>(mp, pl, st) : lut64_nb<4, 8, PB>(mp, pl, st);
        default: return pl.DT == 4 ? lut64_nb<8, 4, PB>(mp, pl, st) : lut64_nb<8, 8, PB>(mp, pl, st);
    }
}

// contiguous rows (128-dim values, 256-codeword LUT, byte codes; MK: with a mask, NV: scores only):
// at most 8 rows per LUT
template <int RP, int VT, bool MK, bool NV, bool HV>
int launch_ct_nb(const MfmaParams& mp, const SsqMfmaPlan& pl, hipStream_t st) {
    switch (mp.a.n_blocks) {
        case 8: return launch<RP, 8, VT, 8, kNC, 0, true, MK, NV, HV>(mp, pl, st);
        case 16: if constexpr (RP <= 8) return launch<RP, 8, VT, 16, kNC, 0, true, MK, NV, HV>(mp, pl, st); break;
        case 32: if constexpr (RP <= 4) return launch<RP, 8, VT, 32, kNC, 0, true, MK, NV, HV>(mp, pl, st); break;
        default: if constexpr (RP <= 2) return launch<RP, 8, VT, 64, kNC, 0, true, MK, NV, HV>(mp, pl, st); break;
    }
    return ssq_fail(SSQ_ERR_UNSUPPORTED, "MFMA decode: LUT of %d rows x %d blocks exceeds LDS", RP, mp.a.n_blocks);
}
template <int VT, bool MK, bool NV = false, bool HV = false>
int launch_ct(const MfmaParams& mp, const SsqMfmaPlan& pl, hipStream_t st) {
    switch (pl.RP) {
        case 1: return launch_ct_nb<1, VT, MK, NV, HV>(mp, pl, st);
        case 2: return launch_ct_nb<2, VT, MK, NV, HV>(mp, pl, st);
        case 4: return launch_ct_nb<4, VT, MK, NV, HV>(mp, pl, st);
        case 8: return launch_ct_nb<8, VT, MK, NV, HV>(mp, pl, st);
        default: return ssq_fail(SSQ_ERR_UNSUPPORTED, "MFMA decode: %d rows per contiguous LUT", pl.RP);
    }
}

}  // namespace

// the instantiation units: the 256-codeword LUT kernel by row count, and the 64-codeword one
#define SSQ_MFMA_UNIT(name) int name(const SsqPagedParams& mp, const SsqMfmaPlan& pl, hipStream_t st)
SSQ_MFMA_UNIT(ssq_mfma_lut_rp1);
SSQ_MFMA_UNIT(ssq_mfma_lut_rp2);
SSQ_MFMA_UNIT(ssq_mfma_lut_rp4);
SSQ_MFMA_UNIT(ssq_mfma_lut_rp8_16);
SSQ_MFMA_UNIT(ssq_mfma_lut64);
SSQ_MFMA_UNIT(ssq_mfma_lut_ct_bf16);
SSQ_MFMA_UNIT(ssq_mfma_lut_ct_f16);
SSQ_MFMA_UNIT(ssq_mfma_lut_ct_bf16_mask);
SSQ_MFMA_UNIT(ssq_mfma_lut_ct_f16_mask);
SSQ_MFMA_UNIT(ssq_mfma_lut_ct_scores);
SSQ_MFMA_UNIT(ssq_mfma_lut_ct_bf16_heavy);
SSQ_MFMA_UNIT(ssq_mfma_lut_ct_f16_heavy);
