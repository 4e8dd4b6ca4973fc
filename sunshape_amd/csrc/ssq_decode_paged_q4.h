// Paged decode with the scores on 4x4 matrix-core blocks (gfx950).  The kernel template; its
// instantiations are spread over ssq_decode_paged_q4_*.hip (compiled in parallel) and dispatched
// from ssq_decode_paged_q4.hip.
//
// Paged decode with the scores on 4x4 matrix-core blocks: for query-row counts whose LUT
// does not fit the LDS (8 query heads per KV head, or 64 blocks of dim 2 at head_dim 128, the
// reference's default 4 bits/dim), and for codebooks other than 256 / 64 codewords.
//
// Same mathematics as the LUT kernels (ssq_decode_mfma.h): scores q_perm . k_hat in fp32
// (triton_kernels.py:381-408, :174-196, summed here in MFMA order, so within fp32 rounding of the
// LUT path), online softmax, probabilities cast to the value dtype before P.V
// (vllm_attn_backend.py:251-252).  Mapping:
//
//   workgroup = 8 waves (two per SIMD) for one (batch, KV head, context split, group of <= 16
//               query rows); the codebook [nb][nc][bd] fp32 sits in LDS (128 KiB at head_dim 128
//               and 256 codewords), so one workgroup per CU.
//   wave      = streams 64-token tiles (4 pages) with its own running (max, sum, O) and one
//               register set: a tile's codes are reloaded for the next tile as soon as its scores
//               are done, its values as soon as its P.V is done; waves merge through LDS at the end.
//   scores    = one token per lane.  v_mfma_f32_4x4x1_16b_f32 computes 16 blocks of 4 rows x 4
//               tokens x 1 dim: with the A operand broadcast from one block (cbsz 4, abid j) every
//               block multiplies the same 4 query rows, so one instruction adds dim k of all 64
//               tokens for 4 rows, and lane l's output VGPR i is row i's score for token l (the
//               lane layout was checked on the device).  Lane 4j + i holds q_perm[row i][16kk + j]
//               in A register kk, so dim 16kk + j is register kk with abid j: head_dim / 16
//               registers per 4 rows.  The B operand is the lane's own token's codeword element,
//               gathered from the LDS codebook bd floats at a time (ds_read_b64 at block_dim 2).
//               Cost per 64-token tile: head_dim x ceil(rows / 4) two-pass MFMAs; the 16x16x4
//               form spends as much on 4 rows as on 16.
//   P.V       = v_mfma_f32_16x16x32_bf16 / _f16 with V fragments straight from the dim-major page
//               (tile_softmax_pv, shared with the LUT kernel).
//
// With CT = true the same kernel reads the reference's contiguous rows (codes [B, Hkv, T, nb], V
// [B, Hkv, T, 128] token-major) at head_dim 128.  The scores are unchanged.  For P.V the matrix
// core's B operand needs 8 consecutive tokens of one dim per lane, and a token-major row gives 8
// consecutive dims of one token.  So lane l loads 16 bytes (dims 8 (l % 16) .. + 7) of each of the
// 8 tokens 32 g + 8 (l / 16) .. + 7 of K group g -- 16 lanes read one 256-byte row, so every load
// is coalesced -- and transposes that 8 x 8 block of 16-bit values inside its own registers (32
// v_perm_b32 per K group).  Fragment e then holds tokens 8 (l / 16) .. + 7 of dim 8 (l % 16) + e:
// the B operand of one 16x16x32 MFMA whose output column l % 16 is dim 8 (l % 16) + e.  The
// A operand (P from the strip) is the paged kernel's.  No LDS buffer, so eight waves fit beside the
// 128 KiB codebook.
#pragma once

#include "ssq_decode_paged.h"

#include <math.h>

#include <type_traits>

#ifndef SSQ_Q4_WAVES
#define SSQ_Q4_WAVES 8
#endif

namespace {

// LDS carve-up (bytes): codebook [NB][nc][BD] fp32, padded to 1 KiB | P strips [waves][RP][64]
// 16-bit (the query rows [RP][KD] fp32 pass through them in the prologue) | pages [split_len/16]
// int32.  The waves' merge reuses the codebook region.
__host__ __device__ constexpr int q4_cb_floats(int KD, int nc) { return (KD * nc + 255) / 256 * 256; }
inline size_t q4_strip_bytes(int RP, int W) { return (size_t)W * RP * kTileTok * 2; }
inline size_t q4_smem(const ssq_decode_args& a, int RP, int split_len, int W) {
    const size_t pages = a.layout == SSQ_PAGED ? (size_t)split_len / kPage * 4 : 0;
    const size_t main = (size_t)q4_cb_floats(a.head_dim, a.n_centroids) * 4 + q4_strip_bytes(RP, W) + pages;
    const size_t merge = (size_t)W * RP * (a.value_dim + 2) * 4;
    return main > merge ? main : merge;
}

// The halves of issue_tile (ssq_decode_paged.h), for the one-register-set pipeline: a tile's codes
// are reloaded as soon as its scores are done, its values as soon as its P.V is done.
template <int NB, int DT, int PB>
__device__ __forceinline__ void issue_codes(const ssq_decode_args& a, const int* pages, int t_begin, int t_end, int tile,
                                            int lane, const uint8_t* cbase, TileRegs<NB, DT, PB>& R) {
    const int last = t_end - 1 - t_begin;
    const int tr = min(tile * kTileTok + lane, last);
    const int page = pages[tr >> 4];
    if constexpr (PB > 0) {
        const uint32_t* prow = reinterpret_cast<const uint32_t*>(cbase) + (int64_t)page * a.c_sb +
                               (int64_t)((t_begin + tr) & 15) * a.c_st;
#pragma unroll
        for (int i = 0; i < pk_words(NB, PB); ++i) R.pk[i] = __builtin_nontemporal_load(prow + i);
    } else if constexpr (NB >= 16) {
        const uint8_t* crow = cbase + (int64_t)page * a.c_sb + (int64_t)((t_begin + tr) & 15) * a.c_st;
#pragma unroll
        for (int i = 0; i < NB / 16; ++i) {
            const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(crow) + i);
            R.c[i] = make_uint4(v.x, v.y, v.z, v.w);
        }
    } else {
        const uint8_t* crow = cbase + (int64_t)page * a.c_sb + (int64_t)((t_begin + tr) & 15) * a.c_st;
        R.c8 = *reinterpret_cast<const uint2*>(crow);
    }
}
template <int NB, int DT, int PB>
__device__ __forceinline__ void issue_values(const ssq_decode_args& a, const int* pages, int t_begin, int t_end, int tile,
                                             int lane, const uint16_t* vbase, TileRegs<NB, DT, PB>& R) {
    const int last = t_end - 1 - t_begin;
    const int kchunk = 8 * (lane >> 4);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        const int r = min(tile * kTileTok + 32 * g + kchunk, last & ~7);
        const uint16_t* src = vbase + (int64_t)pages[r >> 4] * a.v_sb + (r & 15);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) R.v[g][dt] = load_stream(src + (int64_t)(16 * dt) * a.v_st);
    }
}

// Contiguous rows (CT).  cb0 / vb0 (bytes) point at the split's first token of this (batch, KV
// head); lim = the split's last token counted from the tile's first (>= 0).  Lanes and tokens past
// it read that token: a valid row whose probability is 0.  Offsets from the tile's first token are
// 32-bit (the plan keeps 64 tokens' strides below 2^31 bytes), so every load is one uniform base
// plus a lane offset.
template <int NB, int DT, int PB>
__device__ __forceinline__ void issue_codes_ct(const ssq_decode_args& a, int t_begin, int t_end, int tile, int lane,
                                               const uint8_t* cb0, TileRegs<NB, DT, PB>& R) {
    const int rel = tile * kTileTok;
    const int lim = t_end - 1 - t_begin - rel;
    const uint32_t tok = (uint32_t)min(lane, lim);
    if constexpr (PB > 0) {  // c_st counts int32 words
        const uint32_t* prow = reinterpret_cast<const uint32_t*>(cb0) + (int64_t)rel * a.c_st + tok * (uint32_t)a.c_st;
#pragma unroll
        for (int i = 0; i < pk_words(NB, PB); ++i) R.pk[i] = __builtin_nontemporal_load(prow + i);
    } else if constexpr (NB >= 16) {
        const uint8_t* crow = cb0 + (int64_t)rel * a.c_st + tok * (uint32_t)a.c_st;
#pragma unroll
        for (int i = 0; i < NB / 16; ++i) {
            const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(crow) + i);
            R.c[i] = make_uint4(v.x, v.y, v.z, v.w);
        }
    } else {
        R.c8 = *reinterpret_cast<const uint2*>(cb0 + (int64_t)rel * a.c_st + tok * (uint32_t)a.c_st);
    }
}
// R.v[g][i]: dims 8 (lane % 16) .. + 7 of token 32 g + 8 (lane / 16) + i (128-dim rows)
template <int NB, int DT, int PB>
__device__ __forceinline__ void issue_values_ct(const ssq_decode_args& a, int t_begin, int t_end, int tile, int lane,
                                                const uint8_t* vb0, TileRegs<NB, DT, PB>& R) {
    static_assert(DT == 8, "contiguous 4x4-MFMA tiles carry 128-dim values");
    const int rel = tile * kTileTok;
    const int lim = t_end - 1 - t_begin - rel;
    const uint8_t* vtile = vb0 + (int64_t)rel * 2 * a.v_st;
    const uint32_t vst = 2u * (uint32_t)a.v_st, dcol = 16u * (uint32_t)(lane & 15);
    const int k0 = 8 * (lane >> 4);
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t tok = (uint32_t)min(32 * g + k0 + i, lim);
            R.v[g][i] = load_stream(reinterpret_cast<const uint16_t*>(vtile + tok * vst + dcol));
        }
}

// Dim 8 (lane % 16) + E of the 8 tokens in rows v[0..7] (row i = one token's 8 dims, two to a
// dword, the lower dim in the low half): 8 bf16 / f16 values, token j in half j % 2 of dword j / 2.
template <int E>
__device__ __forceinline__ uint4 column8(const uint4 (&v)[8]) {
    constexpr uint32_t sel = (E & 1) ? 0x07060302u : 0x05040100u;  // high or low halves of both words
    auto word = [](const uint4& x) -> uint32_t {
        return (E >> 1) == 0 ? x.x : (E >> 1) == 1 ? x.y : (E >> 1) == 2 ? x.z : x.w;
    };
    return make_uint4(__builtin_amdgcn_perm(word(v[1]), word(v[0]), sel), __builtin_amdgcn_perm(word(v[3]), word(v[2]), sel),
                      __builtin_amdgcn_perm(word(v[5]), word(v[4]), sel), __builtin_amdgcn_perm(word(v[7]), word(v[6]), sel));
}

// P.V of a contiguous tile after tile_probs: per K group g, A = P [16 rows x 32 tokens] from the strip
// (as in tile_softmax_pv), B = the in-register transposes of R.v[g]; acc[e] accumulates dim
// 8 (lane % 16) + e of rows 4 (lane / 16) .. + 3.
template <int RP, int DT, int VT, int NB, int PB>
__device__ __forceinline__ void tile_pv_q4ct(const uint16_t* pstrip, int lane, const TileRegs<NB, DT, PB>& R,
                                             v4f (&acc)[DT]) {
    const int arow = lane & 15;
    const int kchunk = 8 * (lane >> 4);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        uint4 af = make_uint4(0, 0, 0, 0);
        if (arow < RP) af = *reinterpret_cast<const uint4*>(pstrip + arow * kTileTok + 32 * g + kchunk);
        acc[0] = mfma<VT>(af, column8<0>(R.v[g]), acc[0]);
        acc[1] = mfma<VT>(af, column8<1>(R.v[g]), acc[1]);
        acc[2] = mfma<VT>(af, column8<2>(R.v[g]), acc[2]);
        acc[3] = mfma<VT>(af, column8<3>(R.v[g]), acc[3]);
        acc[4] = mfma<VT>(af, column8<4>(R.v[g]), acc[4]);
        acc[5] = mfma<VT>(af, column8<5>(R.v[g]), acc[5]);
        acc[6] = mfma<VT>(af, column8<6>(R.v[g]), acc[6]);
        acc[7] = mfma<VT>(af, column8<7>(R.v[g]), acc[7]);
    }
    __builtin_amdgcn_wave_barrier();
}

// code of block blk for this lane's token (byte rows, or PB-bit codes packed in words)
template <int NB, int DT, int PB>
__device__ __forceinline__ uint32_t token_code(const TileRegs<NB, DT, PB>& R, int blk) {
    if constexpr (PB > 0) {
        constexpr int kVpe = 32 / PB;
        return (R.pk[blk / kVpe] >> ((blk % kVpe) * PB)) & ((1u << PB) - 1u);
    } else {
        const int wi = blk >> 2;
        uint32_t word;
        if constexpr (NB >= 16) {
            const uint4 c = R.c[wi >> 2];
            word = (wi & 3) == 0 ? c.x : (wi & 3) == 1 ? c.y : (wi & 3) == 2 ? c.z : c.w;
        } else {
            word = (wi & 1) ? R.c8.y : R.c8.x;
        }
        return __builtin_amdgcn_ubfe(word, 8 * (blk & 3), 8);
    }
}

// BD consecutive floats from LDS (BD = 1, 2, 4 or 8; 4*BD-byte aligned)
template <int BD>
__device__ __forceinline__ void lds_vec(const float* src, float (&dst)[BD]) {
    if constexpr (BD >= 4) {
#pragma unroll
        for (int i = 0; i < BD; i += 4) {
            const float4 v = *reinterpret_cast<const float4*>(src + i);
            dst[i] = v.x; dst[i + 1] = v.y; dst[i + 2] = v.z; dst[i + 3] = v.w;
        }
    } else if constexpr (BD == 2) {
        const float2 v = *reinterpret_cast<const float2*>(src);
        dst[0] = v.x; dst[1] = v.y;
    } else {
        dst[0] = src[0];
    }
}

// Compile-time loop: f(std::integral_constant<int, I>) for I = B .. E-1 (the MFMA's broadcast block
// id must be an immediate).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// Scores of one tile: s[r] = row r's score for this lane's token.  Codeword gathers are issued one
// batch (KB blocks) ahead of the MFMAs that consume them, so an LDS latency overlaps a batch of
// matrix-core work.  With one row quad, even and odd blocks accumulate into separate chains (two
// independent MFMA dependency chains), added at the end; more quads interleave their own chains.
template <int KB, int NB, int BD, int DT, int PB>
__device__ __forceinline__ void gather_batch(const float* cb, int nc, uint32_t ncm1, const TileRegs<NB, DT, PB>& R,
                                             int b0, float (&ev)[KB][BD]) {
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const int blk = b0 + k;
        const uint32_t code = min(token_code<NB, DT, PB>(R, blk), ncm1);
        lds_vec<BD>(cb + ((uint32_t)blk * (uint32_t)nc + code) * BD, ev[k]);
    }
}

template <int KD, int BD, int R4, int DT, int PB>
__device__ __forceinline__ void tile_scores_q4(const float* cb, int nc, const TileRegs<KD / BD, DT, PB>& R,
                                               const float (&qa)[R4][KD / 16], float (&s)[4 * R4]) {
    constexpr int NB = KD / BD;
    constexpr int KB = BD >= 4 ? 4 : 8;  // blocks gathered per batch
    constexpr int NBATCH = NB / KB;
    static_assert(NB % KB == 0, "blocks per batch must divide the block count");
    const uint32_t ncm1 = (uint32_t)(nc - 1);
    v4f c0[R4], c1[R4];
#pragma unroll
    for (int q = 0; q < R4; ++q) {
        c0[q] = (v4f){0.f, 0.f, 0.f, 0.f};
        c1[q] = (v4f){0.f, 0.f, 0.f, 0.f};
    }
    float ev[2][KB][BD];
    gather_batch<KB, NB, BD, DT, PB>(cb, nc, ncm1, R, 0, ev[0]);
    static_for<0, NBATCH>([&](auto bc) {
        constexpr int bi = decltype(bc)::value;
        constexpr int b0 = bi * KB;
        if constexpr (bi + 1 < NBATCH) gather_batch<KB, NB, BD, DT, PB>(cb, nc, ncm1, R, b0 + KB, ev[(bi + 1) & 1]);
        // keep the next batch's gathers ahead of this batch's MFMAs (the scheduler would otherwise
        // sink each gather to its first use and wait on every one)
        __builtin_amdgcn_sched_barrier(0);
        static_for<0, KB * BD>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            constexpr int k = i / BD, d = i % BD;
            constexpr int blk = b0 + k, kd = blk * BD + d;
            const float e = ev[bi & 1][k][d];
#pragma unroll
            for (int q = 0; q < R4; ++q) {
                if constexpr (R4 == 1 && (blk & 1))
                    c1[q] = __builtin_amdgcn_mfma_f32_4x4x1f32(qa[q][kd >> 4], e, c1[q], 4, kd & 15, 0);
                else
                    c0[q] = __builtin_amdgcn_mfma_f32_4x4x1f32(qa[q][kd >> 4], e, c0[q], 4, kd & 15, 0);
            }
        });
        __builtin_amdgcn_sched_barrier(0);
    });
#pragma unroll
    for (int q = 0; q < R4; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[4 * q + i] = R4 == 1 ? c0[q][i] + c1[q][i] : c0[q][i];
}

// A tile's registers beside its codes and values: the additive mask of each row for this lane's
// token (MK) and the passthrough values of this lane's token as raw bits (HV).
template <int RP, bool MK, int HV>
struct TileExtra {
    float mk[MK ? RP : 1];
    uint32_t pt[HV ? 16 : 1];
};

// Mask and passthrough loads of one tile for this lane's token (the split's last token past its end:
// a valid address; its probability is 0).  Rows past the workgroup's last re-read that row's mask.
// HV 1: the n_hd (8 or 16) values are consecutive 16-bit elements in 16-byte aligned rows, two
// 16-byte loads (the second re-reads the first with 8); HV 2: one load per value (any dtype, any
// slots), all 16 issued under one branch on the dtype.
template <int RP, bool MK, int HV, bool CT>
__device__ __forceinline__ void issue_extra(const MfmaParams& p, const int* pages, int b, int kv, int t_begin, int t_end,
                                            int tile, int lane, TileExtra<RP, MK, HV>& X) {
    if constexpr (MK || HV > 0) {
        const ssq_decode_args& a = p.a;
        const int tr = min(tile * kTileTok + lane, t_end - 1 - t_begin);  // from the split's first token
        const int64_t t = (int64_t)t_begin + tr;
        if constexpr (MK) {
            const int row0 = blockIdx.z * p.rg, nr = min(p.rg, p.rows - row0);
#pragma unroll
            for (int r = 0; r < RP; ++r) {
                const int rr = row0 + min(r, nr - 1);
                const int g = rr / a.q_len, qi = rr - g * a.q_len;
                const int h = kv * p.G + g;
                X.mk[r] = a.mask[(int64_t)b * a.m_sb + (int64_t)h * a.m_sh + (int64_t)qi * a.m_sl + t * a.m_st];
            }
        }
        if constexpr (HV > 0) {
            const int64_t row = CT ? (int64_t)b * a.pt_sb + (int64_t)kv * a.pt_sh + t * a.pt_st
                                   : (int64_t)pages[tr >> 4] * a.pt_sb + (int64_t)kv * a.pt_sh + (int64_t)(t & 15) * a.pt_st;
            if constexpr (HV == 1) {
                const uint4* src = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.pt) + row + p.hoff[0]);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint4 w = src[min(j, p.n_hd / 8 - 1)];
                    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        X.pt[8 * j + 2 * k] = ww[k] & 0xFFFFu;
                        X.pt[8 * j + 2 * k + 1] = ww[k] >> 16;
                    }
                }
            } else {
                // slots past n_hd re-read the last one (compile-time indices into the arguments)
                int hlast = p.hoff[0];
#pragma unroll
                for (int j = 1; j < 16; ++j) hlast = j < p.n_hd ? p.hoff[j] : hlast;
                int64_t idx[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) idx[i] = row + (i < p.n_hd ? p.hoff[i] : hlast);
                if (a.pt_dtype == SSQ_F32) {
                    const uint32_t* f = reinterpret_cast<const uint32_t*>(a.pt);
#pragma unroll
                    for (int i = 0; i < 16; ++i) X.pt[i] = f[idx[i]];
                } else {
                    const uint16_t* h = reinterpret_cast<const uint16_t*>(a.pt);
#pragma unroll
                    for (int i = 0; i < 16; ++i) X.pt[i] = h[idx[i]];
                }
            }
        }
    }
}

// Scores of the passthrough dims and the mask, added to a tile's scores s (whose MFMA pass saw zero
// query values on those dims): one 4x4x1 MFMA per passthrough dim i and row quad q, the A operand
// qh[q] broadcast from block i (lane 4 i + r holds q_perm[row 4 q + r][hdim[i]]), the B operand this
// lane's stored value of dim i.
template <int R4, bool MK, int HV>
__device__ __forceinline__ void tile_extra_scores(const MfmaParams& p, const float (&qh)[R4], const TileExtra<4 * R4, MK, HV>& X,
                                                  float (&s)[4 * R4]) {
    if constexpr (HV > 0) {
        v4f c[R4];
#pragma unroll
        for (int q = 0; q < R4; ++q) c[q] = (v4f){0.f, 0.f, 0.f, 0.f};
        static_for<0, 16>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            if (i < p.n_hd) {  // wave-uniform
                const float x = ssq_bits_to_f32(X.pt[i], p.a.pt_dtype);
#pragma unroll
                for (int q = 0; q < R4; ++q) c[q] = __builtin_amdgcn_mfma_f32_4x4x1f32(qh[q], x, c[q], 4, i, 0);
            }
        });
#pragma unroll
        for (int q = 0; q < R4; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) s[4 * q + i] += c[q][i];
    }
    if constexpr (MK) {
        const int nr = min(p.rg, p.rows - (int)blockIdx.z * p.rg);
#pragma unroll
        for (int r = 0; r < 4 * R4; ++r) s[r] += r < nr ? X.mk[r] : 0.f;
    }
}

// W waves per workgroup: 4 (one per SIMD) keep two tiles in flight per wave in two register sets;
// 8 (two per SIMD, so one wave's matrix-core phase overlaps the other's VALU and LDS phases) keep
// one set, reloading a tile's codes once its scores are done and its values once its P.V is done.
// The LDS (codebook) limits a CU to one workgroup, i.e. W / 4 waves per SIMD: telling the compiler
// so lets it spend registers on loads in flight instead of trimming them for an occupancy the LDS
// never allows.
// MK: an additive mask; HV: passthrough blocks (1: 8 or 16 consecutive 16-bit values per token, 2:
// any layout and dtype); both with byte codes only.
template <int KD, int BD, int R4, int DT, int VT, int PB, int W, bool CT, bool MK, int HV>
__global__ __launch_bounds__(W * SSQ_WAVE) __attribute__((amdgpu_waves_per_eu(W / 4, W / 4)))
void k_decode_paged_q4(const MfmaParams p) {
    static_assert(!CT || (W == 8 && DT == 8), "contiguous rows: 8 waves, 128-dim values");
    static_assert(!(MK || HV) || (W == 8 && PB == 0), "masks and passthrough: 8 waves, byte codes");
    constexpr int kThreads = W * SSQ_WAVE;
    constexpr int kWaves = W;
    constexpr int NB = KD / BD;
    constexpr int RP = 4 * R4;
    constexpr int KQ = KD / 16;  // A registers per row quad
    extern __shared__ __align__(16) float smem[];
    const ssq_decode_args& a = p.a;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bk = blockIdx.x;
    const int split = blockIdx.y;
    const int b = bk / a.num_kv_heads;
    const int kv = bk - b * a.num_kv_heads;
    const int nc = a.n_centroids;
    const int row0 = blockIdx.z * p.rg;       // this workgroup's query rows: row0 .. row0 + nr - 1
    const int nr = min(p.rg, p.rows - row0);  // <= RP
    const int T = CT ? a.seq_len : min(a.seq_lens[b], a.seq_len);
    const int t_begin = split * p.split_len;
    const int t_end = min(T, t_begin + p.split_len);

    float* cb = smem;
    uint8_t* strips = reinterpret_cast<uint8_t*>(smem + q4_cb_floats(KD, nc));
    uint16_t* pstrip = reinterpret_cast<uint16_t*>(strips) + wave * RP * kTileTok;
    int* pages = reinterpret_cast<int*>(strips + (size_t)kWaves * RP * kTileTok * 2);  // paged only

    // ---- prologue: block-table slice, this lane's permutation entries, the query rows (scaled,
    // unpermuted) through LDS into the A registers
    const int32_t* btab = CT ? nullptr : a.block_table + (int64_t)b * a.bt_sb + t_begin / kPage;
    const int n_pages = !CT && t_end > t_begin ? (t_end - t_begin + kPage - 1) / kPage : 0;
    for (int i = tid; i < n_pages; i += kThreads) pages[i] = btab[i];
    const int64_t* perm = a.perm + (int64_t)kv * a.perm_sh;
    const int qi4 = lane & 3, qj = lane >> 2;
    int64_t pj[KQ];
#pragma unroll
    for (int kk = 0; kk < KQ; ++kk) pj[kk] = perm[16 * kk + qj];
    float* qs = reinterpret_cast<float*>(strips);  // [RP][KD] fp32: RP * KD * 4 <= the strips' RP * 512 bytes
    {
        constexpr int kQE = (RP * KD + kThreads - 1) / kThreads;
        int64_t src[kQE];
        bool ok[kQE];
#pragma unroll
        for (int k = 0; k < kQE; ++k) {
            const int e = tid + k * kThreads;
            const int r = e / KD, j = e - r * KD;
            ok[k] = e < RP * KD && r < nr;
            src[k] = 0;  // rows past nr read element 0 and are zeroed
            if (ok[k]) {
                const int g = (row0 + r) / a.q_len, qi = row0 + r - g * a.q_len;
                const int h = kv * p.G + g;
                src[k] = (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)qi * a.q_sl + j;
            }
        }
        float qv[kQE];
        ssq_load_elems(a.q, a.q_dtype, src, qv);
#pragma unroll
        for (int k = 0; k < kQE; ++k) {
            const int e = tid + k * kThreads;
            if (e < RP * KD) qs[e] = !ok[k] ? 0.f : a.has_scale ? ssq_round_to(qv[k] * a.scale, a.q_dtype) : qv[k];
        }
    }
    __syncthreads();  // qs and pages written
    float qa[R4][KQ];
#pragma unroll
    for (int q = 0; q < R4; ++q)
#pragma unroll
        for (int kk = 0; kk < KQ; ++kk) {
            qa[q][kk] = qs[(4 * q + qi4) * KD + (int)min((uint64_t)pj[kk], (uint64_t)(KD - 1))];
            // passthrough blocks score from their stored values (tile_extra_scores): no codeword term
            if constexpr (HV > 0)
                if ((a.heavy_mask[0] >> ((16 * kk + qj) / BD)) & 1ull) qa[q][kk] = 0.f;
        }
    // the query rows at the passthrough dims: lane 4 j + r holds q_perm[row 4 q + r][hdim[j]] (j < n_hd)
    float qh[R4];  // (unused without passthrough)
    if constexpr (HV > 0) {
        int hd = 0;  // lanes past the last passthrough dim keep dim 0 (their query value is not used)
#pragma unroll
        for (int j = 0; j < 16; ++j) hd = j == qj && j < p.n_hd ? p.hdim[j] : hd;
        const int pd = (int)min((uint64_t)perm[hd], (uint64_t)(KD - 1));
#pragma unroll
        for (int q = 0; q < R4; ++q) qh[q] = qj < p.n_hd ? qs[(4 * q + qi4) * KD + pd] : 0.f;
    }
    __syncthreads();  // every wave has its A registers: the strips are free

    const uint16_t* vbase = reinterpret_cast<const uint16_t*>(a.v) + (int64_t)kv * a.v_sh + (int64_t)(lane & 15) * a.v_st;
    const uint8_t* cbase = PB > 0 ? reinterpret_cast<const uint8_t*>(reinterpret_cast<const uint32_t*>(a.codes) +
                                                                     (int64_t)kv * a.c_sh)
                                  : a.codes + (int64_t)kv * a.c_sh;
    // contiguous rows: the split's first token of this (batch, KV head), in bytes
    const uint8_t* cb0 = PB > 0 ? reinterpret_cast<const uint8_t*>(reinterpret_cast<const uint32_t*>(a.codes) +
                                                                   (int64_t)b * a.c_sb + (int64_t)kv * a.c_sh +
                                                                   (int64_t)t_begin * a.c_st)
                                : a.codes + (int64_t)b * a.c_sb + (int64_t)kv * a.c_sh + (int64_t)t_begin * a.c_st;
    const uint8_t* vb0 = reinterpret_cast<const uint8_t*>(a.v) +
                         2 * ((int64_t)b * a.v_sb + (int64_t)kv * a.v_sh + (int64_t)t_begin * a.v_st);
    const int n_tiles = (t_end - t_begin + kTileTok - 1) / kTileTok;
    const int last_tile = n_tiles > 0 ? n_tiles - 1 : 0;
    TileRegs<NB, DT, PB> RA, RB;
    TileExtra<RP, MK, HV> XA;
    int tile = wave;
    if (n_tiles > 0) {
        if constexpr (CT) {
            issue_codes_ct<NB, DT, PB>(a, t_begin, t_end, min(tile, last_tile), lane, cb0, RA);
            issue_values_ct<NB, DT, PB>(a, t_begin, t_end, min(tile, last_tile), lane, vb0, RA);
        } else {
            issue_tile<NB, DT, PB>(a, pages, t_begin, t_end, min(tile, last_tile), lane, cbase, vbase, RA);
        }
        issue_extra<RP, MK, HV, CT>(p, pages, b, kv, t_begin, t_end, min(tile, last_tile), lane, XA);
    }
    (void)RB;
    // the codebook goes global -> LDS directly: 1 KiB chunks, lane l's 16 bytes at chunk + 16 l;
    // the tail chunk's lanes past the end re-read the last float4 into the padding
    {
        const float* cent = a.cent + (int64_t)kv * a.cent_sh;
        const int n4 = KD * nc / 4;
        const int n_chunks = (n4 + 63) / 64;
        for (int c = wave; c < n_chunks; c += kWaves) {
            const int i = min(c * 64 + lane, n4 - 1);
            __builtin_amdgcn_global_load_lds(cent + 4 * i, (__attribute__((address_space(3))) void*)(cb + 256 * c), 16,
                                             0, 0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's codebook chunks (and its first tile) have landed
    __syncthreads();

    // ---- stream tiles, two in flight per wave (A/B register sets)
    float m_run[RP], l_lane[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) { m_run[r] = -INFINITY; l_lane[r] = 0.f; }
    v4f acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = (v4f){0.f, 0.f, 0.f, 0.f};
    if constexpr (CT) {
        // one register set, every load unconditional (clamped to the last tile), as below
        while (tile < n_tiles) {
            const int next = min(tile + kWaves, last_tile);
            float s[RP];
            tile_scores_q4<KD, BD, R4, DT, PB>(cb, nc, RA, qa, s);
            tile_extra_scores<R4, MK, HV>(p, qh, XA, s);
            issue_codes_ct<NB, DT, PB>(a, t_begin, t_end, next, lane, cb0, RA);
            issue_extra<RP, MK, HV, CT>(p, pages, b, kv, t_begin, t_end, next, lane, XA);
            tile_probs<RP, DT, VT>(p, pstrip, b, kv, t_begin + tile * kTileTok, t_end, lane, s, m_run, l_lane, acc);
            tile_pv_q4ct<RP, DT, VT, NB, PB>(pstrip, lane, RA, acc);
            issue_values_ct<NB, DT, PB>(a, t_begin, t_end, next, lane, vb0, RA);
            tile += kWaves;
        }
    } else if constexpr (W == 4) {
        static_assert(!MK && HV == 0, "4-wave build: no mask or passthrough variants");
        while (tile < n_tiles) {
            issue_tile<NB, DT, PB>(a, pages, t_begin, t_end, min(tile + kWaves, last_tile), lane, cbase, vbase, RB);
            {
                float s[RP];
                tile_scores_q4<KD, BD, R4, DT, PB>(cb, nc, RA, qa, s);
                tile_softmax_pv<RP, DT, VT, NB, PB>(p, pstrip, b, kv, t_begin + tile * kTileTok, t_end, lane, s, RA,
                                                    m_run, l_lane, acc);
            }
            tile += kWaves;
            if (tile >= n_tiles) break;
            issue_tile<NB, DT, PB>(a, pages, t_begin, t_end, min(tile + kWaves, last_tile), lane, cbase, vbase, RA);
            {
                float s[RP];
                tile_scores_q4<KD, BD, R4, DT, PB>(cb, nc, RB, qa, s);
                tile_softmax_pv<RP, DT, VT, NB, PB>(p, pstrip, b, kv, t_begin + tile * kTileTok, t_end, lane, s, RB,
                                                    m_run, l_lane, acc);
            }
            tile += kWaves;
        }
    } else {
        // one register set: every load is issued unconditionally (clamped to the last tile), so the
        // queue of outstanding loads is the same on every path
        while (tile < n_tiles) {
            const int next = min(tile + kWaves, last_tile);
            float s[RP];
            tile_scores_q4<KD, BD, R4, DT, PB>(cb, nc, RA, qa, s);
            tile_extra_scores<R4, MK, HV>(p, qh, XA, s);
            issue_codes<NB, DT, PB>(a, pages, t_begin, t_end, next, lane, cbase, RA);
            issue_extra<RP, MK, HV, CT>(p, pages, b, kv, t_begin, t_end, next, lane, XA);
            tile_softmax_pv<RP, DT, VT, NB, PB>(p, pstrip, b, kv, t_begin + tile * kTileTok, t_end, lane, s, RA, m_run,
                                                l_lane, acc);
            issue_values<NB, DT, PB>(a, pages, t_begin, t_end, next, lane, vbase, RA);
            tile += kWaves;
        }
    }

    // ---- merge the waves' (m, l, O) through LDS (the codebook is no longer needed)
    float l_w[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) l_w[r] = wave_sum(l_lane[r]);
    __syncthreads();
    float* mbuf = smem;                // [waves][RP]
    float* lbuf = mbuf + kWaves * RP;  // [waves][RP]
    float* obuf = lbuf + kWaves * RP;  // [waves][RP][Dv]
    constexpr int Dv = DT * 16;
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RP; ++r) { mbuf[wave * RP + r] = m_run[r]; lbuf[wave * RP + r] = l_w[r]; }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 4 * (lane >> 4) + i;
        if (row < RP) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                // contiguous rows: accumulator dt holds dim 8 (lane % 16) + dt; pages: dim 16 dt + lane % 16
                const int dim = CT ? 8 * (lane & 15) + dt : 16 * dt + (lane & 15);
                obuf[((size_t)wave * RP + row) * Dv + dim] = acc[dt][i];
            }
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


// waves per workgroup for this instantiation (see k_decode_paged_q4)
template <int KD, int BD, int R4, int DT>
constexpr int q4_waves() { return SSQ_Q4_WAVES; }

template <int KD, int BD, int R4, int DT, int VT, int PB, bool CT, bool MK, int HV>
int launch_q4(const MfmaParams& mp, const dim3& grid, size_t, hipStream_t st) {
    constexpr int W = q4_waves<KD, BD, R4, DT>();
    auto kern = k_decode_paged_q4<KD, BD, R4, DT, VT, PB, W, CT, MK, HV>;
    int rc = ssq_allow_lds((const void*)kern, (int)kMaxSmem, "hipFuncSetAttribute(decode_paged_q4)");
    if (rc) return rc;
    const size_t smem = q4_smem(mp.a, 4 * R4, mp.split_len, W);
    if (smem > kMaxSmem) return ssq_fail(SSQ_ERR_UNSUPPORTED, "4x4-MFMA decode: %zu bytes of LDS", smem);
    hipLaunchKernelGGL(kern, grid, dim3(W * SSQ_WAVE), smem, st, mp);
    return ssq_check_hip(hipGetLastError(), "k_decode_paged_q4 launch");
}
template <int KD, int BD, int R4, int VT, int PB, bool CT, bool MK, int HV>
int q4_dt(const MfmaParams& mp, int DT, const dim3& grid, size_t smem, hipStream_t st) {
    if constexpr (CT) {  // contiguous rows: 128-dim values only
        return DT == 8 ? launch_q4<KD, BD, R4, 8, VT, PB, true, MK, HV>(mp, grid, smem, st)
                       : ssq_fail(SSQ_ERR_UNSUPPORTED, "4x4-MFMA decode: contiguous rows need 128-dim values");
    } else {
        return DT == 4 ? launch_q4<KD, BD, R4, 4, VT, PB, false, MK, HV>(mp, grid, smem, st)
                       : launch_q4<KD, BD, R4, 8, VT, PB, false, MK, HV>(mp, grid, smem, st);
    }
}
template <int KD, int BD, int VT, int PB, bool CT, bool MK, int HV>
int q4_r4(const MfmaParams& mp, int R4, int DT, const dim3& grid, size_t smem, hipStream_t st) {
    switch (R4) {
        case 1: return q4_dt<KD, BD, 1, VT, PB, CT, MK, HV>(mp, DT, grid, smem, st);
        case 2: return q4_dt<KD, BD, 2, VT, PB, CT, MK, HV>(mp, DT, grid, smem, st);
        case 3: return q4_dt<KD, BD, 3, VT, PB, CT, MK, HV>(mp, DT, grid, smem, st);
        default: return q4_dt<KD, BD, 4, VT, PB, CT, MK, HV>(mp, DT, grid, smem, st);
    }
}
// every instantiation for one head_dim, value dtype, code width and layout (CT: contiguous rows), with
// a mask (MK) and passthrough blocks (HV) or without
template <int KD, int VT, int PB, bool CT = false, bool MK = false, int HV = 0>
int q4_dispatch(const MfmaParams& mp, int R4, int DT, const dim3& grid, size_t smem, hipStream_t st) {
    switch (mp.a.block_dim) {
        case 1: if constexpr (KD <= 64) return q4_r4<KD, 1, VT, PB, CT, MK, HV>(mp, R4, DT, grid, smem, st); break;
        case 2: return q4_r4<KD, 2, VT, PB, CT, MK, HV>(mp, R4, DT, grid, smem, st);
        case 4: return q4_r4<KD, 4, VT, PB, CT, MK, HV>(mp, R4, DT, grid, smem, st);
        case 8: return q4_r4<KD, 8, VT, PB, CT, MK, HV>(mp, R4, DT, grid, smem, st);
        default: break;
    }
    return ssq_fail(SSQ_ERR_UNSUPPORTED, "4x4-MFMA decode: block_dim %d at head_dim %d", mp.a.block_dim, KD);
}
// the mask / passthrough variants of one head_dim, value dtype and layout (byte codes): passthrough
// values loaded as vectors (HV 1) without a mask, element by element (HV 2) otherwise
template <int KD, int VT, bool CT>
int q4_dispatch_mixed(const MfmaParams& mp, int R4, int DT, const dim3& grid, size_t smem, hipStream_t st) {
    const bool mk = mp.a.mask != nullptr;
    const bool hv = mp.a.heavy_mask[0] != 0;
    if (!hv) return q4_dispatch<KD, VT, 0, CT, true, 0>(mp, R4, DT, grid, smem, st);
    if (mk) return q4_dispatch<KD, VT, 0, CT, true, 2>(mp, R4, DT, grid, smem, st);
    if (mp.pt_vec) return q4_dispatch<KD, VT, 0, CT, false, 1>(mp, R4, DT, grid, smem, st);
    return q4_dispatch<KD, VT, 0, CT, false, 2>(mp, R4, DT, grid, smem, st);
}

}  // namespace

// the instantiation units (ssq_decode_paged_q4_<head_dim>_<value dtype>_<codes>.hip)
#define SSQ_Q4_UNIT(name) \
    int name(const SsqPagedParams& mp, int R4, int DT, const dim3& grid, size_t smem, hipStream_t st)
SSQ_Q4_UNIT(ssq_q4_64_bf16_bytes);
SSQ_Q4_UNIT(ssq_q4_64_bf16_packed);
SSQ_Q4_UNIT(ssq_q4_64_f16_bytes);
SSQ_Q4_UNIT(ssq_q4_64_f16_packed);
SSQ_Q4_UNIT(ssq_q4_128_bf16_bytes);
SSQ_Q4_UNIT(ssq_q4_128_bf16_packed);
SSQ_Q4_UNIT(ssq_q4_128_f16_bytes);
SSQ_Q4_UNIT(ssq_q4_128_f16_packed);
SSQ_Q4_UNIT(ssq_q4ct_128_bf16_bytes);
SSQ_Q4_UNIT(ssq_q4ct_128_bf16_packed);
SSQ_Q4_UNIT(ssq_q4ct_128_f16_bytes);
SSQ_Q4_UNIT(ssq_q4ct_128_f16_packed);
SSQ_Q4_UNIT(ssq_q4_64_bf16_mixed);
SSQ_Q4_UNIT(ssq_q4_64_f16_mixed);
SSQ_Q4_UNIT(ssq_q4_128_bf16_mixed);
SSQ_Q4_UNIT(ssq_q4_128_f16_mixed);
SSQ_Q4_UNIT(ssq_q4ct_128_bf16_mixed);
SSQ_Q4_UNIT(ssq_q4ct_128_f16_mixed);
