// Fused VQ-key decode (and scores) over the reference's contiguous layout on the matrix cores: the
// kernel template.  Its instantiations are spread over ssq_decode_contig_*.hip (compiled in
// parallel) and dispatched from ssq_decode_contig.hip.
//
// Same mathematics as the other decode kernels (q scaled in its own dtype, softmax in fp32, the
// probabilities cast to the value dtype before P.V: vllm_attn_backend.py:232-252), mapped for
// contiguous token-major values [B, Hkv, T, Dv] and head_dim 64:
//
//   scores = one token per lane.  v_mfma_f32_4x4x1_16b_f32 computes 16 blocks of 4 rows x 4 tokens
//            x 1 dim; with the A operand broadcast from one block (cbsz 4, abid j) every block
//            multiplies the same 4 query rows, so one instruction adds dim k of all 64 tokens for 4
//            rows, and lane l's output register i is row i's score for token l.  Lane 4j + i holds
//            q_perm[row 4q + i][16kk + j] (scaled) in A register kk of row quad q, so dim 16kk + j is
//            register kk with abid j.  The B operand is the lane's own codeword element, gathered
//            from the codebook staged in LDS block_dim floats at a time; the lane's codes stay in
//            registers.  Passthrough (heavy) dims add their stored values in a second pass.  fp32
//            products and sums, one dim per step in ascending order (within fp32 rounding of the LUT
//            kernels' block-by-block sums).  Cost per 64-token tile: 64 x ceil(rows / 4) MFMAs.
//   P.V    = v_mfma_f32_16x16x32_bf16 (_f16): A = P [16 rows x 32 tokens] from a per-wave LDS strip;
//            B = V [32 tokens x 16 dims].  V tiles are copied to LDS with coalesced 16-byte loads
//            and read back transposed with ds_read_b64_tr_b16: within each 16-lane group, lane l
//            addresses V[t0 + l/4][n0 + 4*(l%4) .. +3] and receives V[t0 .. t0+3][n0 + l], so two
//            reads give a lane its 8 consecutive tokens of one dim.
//
// Codes arrive as byte rows or as 4- / 6-bit codes packed into int32 words
// (sunshape/triton_kernels.py:250-266), extracted in registers.
//
// workgroup = 8 waves (4 where the LDS or the registers do not allow 8) for one (batch, KV head,
// context split); each wave streams 64-token tiles with its own running (max, sum, O), the next
// tiles' loads in flight; waves merge through LDS at the end.
#pragma once

#include "ssq_common.h"

#include <math.h>

#include <type_traits>

// Parameters of one contiguous decode launch (shared type: the host code and every instantiation
// unit fill or read it)
// Codes packed at a width the kernel takes at run time (PB < 0): bits per code, codes per int32
// word (vpe = 32 / bits), words per token row, and mul = ceil(65536 / vpe), so that blk / vpe =
// (blk * mul) >> 16 exactly for blk < 64.
struct SsqPackFmt {
    uint32_t bits, vpe, mul, nw;
};

struct SsqContigParams {
    ssq_decode_args a;
    int G, rows, split_len, n_splits;
    float* ws_o;
    float* ws_m;
    float* ws_l;
    // passthrough dims (SunShape-Mixed): the token record element and the permuted head dim of
    // heavy dim idx (blocks ascending, then d); n_hd of them
    int n_hd;
    int pt_vec;  // 1: the 8 passthrough values are contiguous 16-bit elements from slot 0, 16-byte aligned
    int hoff[16];
    int hdim[16];
    SsqPackFmt pk;  // PB < 0 variants
};

// Launch shape chosen by the host: value tiles of 16 dims, waves per workgroup, row quads
struct SsqContigPlan {
    int DT, split_len, n_splits, waves, r4;
    size_t smem, ws_bytes;
};

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr int kTile = 64;  // tokens per wave iteration
constexpr int kD = 64;     // head_dim served
constexpr int kHP = 16;    // passthrough (heavy-block) dims per token served
constexpr size_t kMaxSmem = 160 * 1024;

// per-wave LDS region (bytes): V tile [64][Dv] (16-bit) | P strip [16][64] (16-bit).  The scaled
// query rows [16][64] fp32 pass through the V region in the prologue.
__host__ __device__ constexpr int wave_v_bytes(int DT) { return kTile * DT * 16 * 2; }
__host__ __device__ constexpr int wave_bytes(int DT) { return wave_v_bytes(DT) + 16 * kTile * 2; }
// codebook region: [NB][nc][BD] fp32, padded to whole 1 KB chunks (one direct-to-LDS wave load each)
__host__ __device__ constexpr int cb_floats(int nc) { return (16 * nc + 63) / 64 * 256; }
inline size_t contig_smem(const ssq_decode_args& a, int DT, int waves) {
    const size_t cb = (size_t)cb_floats(a.n_centroids) * 4;
    const size_t main = cb + (size_t)waves * wave_bytes(DT);
    const size_t merge = (size_t)waves * 16 * (16 * DT + 2) * 4;
    return main > merge ? main : merge;
}

__device__ __forceinline__ uint4 ld16(const void* p) {
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

template <int VT>
__device__ __forceinline__ uint32_t to_vt16(float x) {
    return VT == SSQ_BF16 ? ssq_f32_to_bf16(x) : ssq_f32_to_f16(x);
}

template <int VT>
__device__ __forceinline__ v4f mfma_pv(const uint4& a, const uint4& b, v4f c) {
    if (VT == SSQ_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0,
                                                       0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
}

template <int CTL>
__device__ __forceinline__ float dpp_ror(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTL, 0xF, 0xF, false));
}
// max / sum over the wave's 64 lanes (every lane receives the result)
__device__ __forceinline__ float wave_max64(float v) {
    v = fmaxf(v, dpp_ror<0x121>(v)); v = fmaxf(v, dpp_ror<0x122>(v));
    v = fmaxf(v, dpp_ror<0x124>(v)); v = fmaxf(v, dpp_ror<0x128>(v));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ float wave_sum64(float v) {
    v += dpp_ror<0x121>(v); v += dpp_ror<0x122>(v);
    v += dpp_ror<0x124>(v); v += dpp_ror<0x128>(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// packed code rows (PB bits per code, 32 / PB codes per little-endian int32 word, the low bits
// first; sunshape/triton_kernels.py:250-266): int32 words per row
// int32 words per token row of PB-bit codes; PB < 0 (width at run time): room for 7-bit codes,
// the widest below a byte
__host__ __device__ constexpr int pk_words(int NB, int PB) {
    return PB > 0 ? (NB + 32 / PB - 1) / (32 / PB) : PB < 0 ? (NB + 3) / 4 : 1;
}

// Bits of N elements of a tensor of dtype dt with no branch on the dtype (straight-line loads keep
// the compiler's load-counter waits exact, so converting them later does not wait for loads issued
// after them): two 16-bit loads per element, the low and high halves of an fp32 element or the same
// 16-bit element twice.  Every idx[i] must be a valid element offset.
template <int N>
__device__ __forceinline__ void load_halves(const void* p, int dt, const int64_t (&idx)[N], uint32_t (&lo)[N],
                                            uint32_t (&hi)[N]) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    const int64_t w = dt == SSQ_F32 ? 2 : 1;  // 16-bit words per element
#pragma unroll
    for (int i = 0; i < N; ++i) {
        lo[i] = h[idx[i] * w];
        hi[i] = h[idx[i] * w + (w - 1)];
    }
}
// the element as fp32 from its halves, by selects on the (uniform) dtype
__device__ __forceinline__ float halves_to_f32(uint32_t lo, uint32_t hi, int dt) {
    const float f32 = __uint_as_float((hi << 16) | lo);
    const float bf = ssq_bf16_to_f32(lo);
    const float f16 = ssq_f16_to_f32(lo);
    return dt == SSQ_F32 ? f32 : dt == SSQ_BF16 ? bf : f16;
}
// x rounded to dtype dt and back (ssq_round_to), by selects
__device__ __forceinline__ float round_to_sel(float x, int dt) {
    const float bf = ssq_bf16_to_f32(ssq_f32_to_bf16(x));
    const float f16 = ssq_f16_to_f32(ssq_f32_to_f16(x));
    return dt == SSQ_F32 ? x : dt == SSQ_BF16 ? bf : f16;
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

// registers of one 64-token tile in flight, lane = token: its 16-byte V chunks (row-major tile
// chunks, for the LDS copy), its code row (bytes, or PB-bit codes in words), its passthrough values
// and its additive-mask values for the RP query rows.
// HV: passthrough values per token: 0 none; 1 up to kHP values, one load each (any dtype and slot
// layout); 2 exactly 8 contiguous 16-bit values from slot 0, one 16-byte load
template <int NB, int DT, int HV, bool MK, int PB, int RP>
struct Tile {
    uint4 v[2 * DT];
    uint4 c[NB >= 16 ? NB / 16 : 1];
    uint2 c8;
    uint32_t pk[pk_words(NB, PB)];
    uint32_t h[HV == 1 ? kHP : HV == 2 ? 4 : 1];  // raw bits; converted at the passthrough pass
    float mk[MK ? RP : 1];                        // additive mask [row r][this lane's token]
};

// Loads are unconditional; tokens past the split's end re-read the last token's row (valid memory;
// such tokens get p = 0 and are never scored).  The values and the rest are issued separately: a
// tile's values are reloaded as soon as they are in LDS, its codes once its scores are done.
template <int NB, int DT, int HV, bool MK, int PB, int RP>
__device__ __forceinline__ void issue_values(const SsqContigParams& p, int b, int kv, int t0, int t_end, int lane,
                                             Tile<NB, DT, HV, MK, PB, RP>& R) {
    const ssq_decode_args& a = p.a;
    // a wave-uniform base at the tile's first token and 32-bit lane offsets (the host checks that
    // a tile spans less than 2^31 elements), so each load is a scalar base plus one offset register
    const uint16_t* vt = reinterpret_cast<const uint16_t*>(a.v) + (int64_t)b * a.v_sb + (int64_t)kv * a.v_sh +
                         (int64_t)t0 * a.v_st;
    const int last = t_end - 1 - t0;  // tokens past it re-read the last one
    constexpr int kRowChunks = 2 * DT;  // 16-byte chunks per token row (Dv = 16 * DT)
#pragma unroll
    for (int i = 0; i < 2 * DT; ++i) {
        const int chunk = i * SSQ_WAVE + lane;  // chunk of the tile, row-major
        const uint32_t off = (uint32_t)min(chunk / kRowChunks, last) * (uint32_t)a.v_st + (chunk % kRowChunks) * 8;
        R.v[i] = ld16(reinterpret_cast<const uint8_t*>(vt) + 2u * off);  // a 32-bit byte offset
    }
}
template <int NB, int DT, int HV, bool MK, int PB, int RP>
__device__ __forceinline__ void issue_codes(const SsqContigParams& p, int b, int kv, int t0, int t_end, int lane,
                                            Tile<NB, DT, HV, MK, PB, RP>& R) {
    const ssq_decode_args& a = p.a;
    const int tc = min(t0 + lane, t_end - 1);
    const uint32_t rel = (uint32_t)(tc - t0);  // this lane's token within the tile (32-bit offsets below)
    if constexpr (MK) {  // rows past the query rows re-read the last row (never added)
#pragma unroll
        for (int r = 0; r < RP; ++r) {
            const int rr = min(r, p.rows - 1);
            const int gq = rr / a.q_len, qi = rr - gq * a.q_len;
            const int h = kv * p.G + gq;
            R.mk[r] = a.mask[(int64_t)b * a.m_sb + (int64_t)h * a.m_sh + (int64_t)qi * a.m_sl + (int64_t)tc * a.m_st];
        }
    }
    if constexpr (HV == 1) {
        const int64_t pb = (int64_t)b * a.pt_sb + (int64_t)kv * a.pt_sh + (int64_t)tc * a.pt_st;
#pragma unroll
        for (int i = 0; i < kHP; ++i) R.h[i] = ssq_load_bits(a.pt, a.pt_dtype, pb + p.hoff[i]);  // hoff clamped
    } else if constexpr (HV == 2) {
        const uint16_t* pt0 = reinterpret_cast<const uint16_t*>(a.pt) + (int64_t)b * a.pt_sb + (int64_t)kv * a.pt_sh +
                              (int64_t)t0 * a.pt_st;
        const uint4 w = ld16(reinterpret_cast<const uint8_t*>(pt0) + 2u * (rel * (uint32_t)a.pt_st));
        R.h[0] = w.x; R.h[1] = w.y; R.h[2] = w.z; R.h[3] = w.w;
    }
    if constexpr (PB) {  // packed rows: strides count int32 words (one row address, word offsets)
        const uint32_t* prow = reinterpret_cast<const uint32_t*>(a.codes) + (int64_t)b * a.c_sb +
                               (int64_t)kv * a.c_sh + (int64_t)tc * a.c_st;
#pragma unroll
        for (int i = 0; i < pk_words(NB, PB); ++i) {
            // width at run time: the row has p.pk.nw words, the rest of the registers re-read its last
            const int wi = PB > 0 ? i : min(i, (int)p.pk.nw - 1);
            R.pk[i] = __builtin_nontemporal_load(prow + wi);
        }
    } else {
        const uint8_t* c0 = a.codes + (int64_t)b * a.c_sb + (int64_t)kv * a.c_sh + (int64_t)t0 * a.c_st;
        const uint32_t roff = rel * (uint32_t)a.c_st;
        if constexpr (NB >= 16) {
#pragma unroll
            for (int i = 0; i < NB / 16; ++i) R.c[i] = ld16(c0 + roff + 16 * i);
        } else {
            R.c8 = *reinterpret_cast<const uint2*>(c0 + roff);
        }
    }
}

// code of block blk for this lane's token (f: the packing of a run-time width, PB < 0)
template <int NB, int DT, int HV, bool MK, int PB, int RP>
__device__ __forceinline__ uint32_t token_code(const Tile<NB, DT, HV, MK, PB, RP>& R, int blk, const SsqPackFmt& f) {
    if constexpr (PB > 0) {
        constexpr int kVpe = 32 / PB;
        return (R.pk[blk / kVpe] >> ((blk % kVpe) * PB)) & ((1u << PB) - 1u);
    } else if constexpr (PB < 0) {  // word and shift are wave-uniform: a register index, not a load
        const uint32_t w = ((uint32_t)blk * f.mul) >> 16;
        const uint32_t sh = ((uint32_t)blk - w * f.vpe) * f.bits;
        uint32_t words[pk_words(NB, PB)];  // a local copy, indexed in registers
#pragma unroll
        for (int i = 0; i < pk_words(NB, PB); ++i) words[i] = R.pk[i];
        return (words[w] >> sh) & ((1u << f.bits) - 1u);
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

template <int KB, int BD, class T>
__device__ __forceinline__ void gather_batch(const float* cb, int nc, uint32_t ncm1, const T& R, int b0,
                                             const SsqPackFmt& f, float (&ev)[KB][BD]) {
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const int blk = b0 + k;
        const uint32_t code = min(token_code(R, blk, f), ncm1);
        lds_vec<BD>(cb + ((uint32_t)blk * (uint32_t)nc + code) * BD, ev[k]);
    }
}

// Scores of one tile: s[4q + i] = row 4q+i's score for this lane's token.  Codeword gathers are
// issued one batch (KB blocks) ahead of the MFMAs that consume them, so an LDS latency overlaps a
// batch of matrix-core work.  With one row quad, even and odd blocks accumulate into separate
// chains (two independent MFMA dependency chains), added at the end; more quads interleave their
// own chains.  Heavy blocks' A values are zero; their dims come from the passthrough pass.
template <int BD, int R4, int NB, int DT, int HV, bool MK, int PB, int RP>
__device__ __forceinline__ void tile_scores(const float* cb, int nc, const Tile<NB, DT, HV, MK, PB, RP>& R,
                                            const float (&qa)[R4][kD / 16], const float (&qh)[R4], int n_hd,
                                            int pt_dtype, const SsqPackFmt& f, float (&s)[RP]) {
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
    gather_batch<KB, BD>(cb, nc, ncm1, R, 0, f, ev[0]);
    static_for<0, NBATCH>([&](auto bc) {
        constexpr int bi = decltype(bc)::value;
        constexpr int b0 = bi * KB;
        if constexpr (bi + 1 < NBATCH) gather_batch<KB, BD>(cb, nc, ncm1, R, b0 + KB, f, ev[(bi + 1) & 1]);
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
    if constexpr (HV != 0) {  // passthrough pass: B = this token's stored value of heavy dim j
        static_for<0, (HV == 2 ? 8 : kHP)>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            if (HV == 2 || j < n_hd) {  // wave-uniform
                uint32_t bits;
                if constexpr (HV == 2) bits = (R.h[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
                else bits = R.h[j];
                const float hvl = ssq_bits_to_f32(bits, pt_dtype);
#pragma unroll
                for (int q = 0; q < R4; ++q) c0[q] = __builtin_amdgcn_mfma_f32_4x4x1f32(qh[q], hvl, c0[q], 4, j, 0);
            }
        });
    }
#pragma unroll
    for (int q = 0; q < R4; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[4 * q + i] = R4 == 1 ? c0[q][i] + c1[q][i] : c0[q][i];
}

// Codebook staging through registers: float4 (round * K + i) * 64 W + tid, clamped to the last one
template <int K, int W>
__device__ __forceinline__ void cb_load(const v4u* src, int n4, int tid, int round, v4u (&r)[K]) {
#pragma unroll
    for (int i = 0; i < K; ++i) r[i] = src[min((round * K + i) * 64 * W + tid, n4 - 1)];
}
template <int K, int W>
__device__ __forceinline__ void cb_store(float* cb, int n4, int tid, int round, const v4u (&r)[K]) {
#pragma unroll
    for (int i = 0; i < K; ++i) reinterpret_cast<v4u*>(cb)[min((round * K + i) * 64 * W + tid, n4 - 1)] = r[i];
}

// Waves per workgroup: 8 (two per SIMD: one wave's matrix-core phase overlaps the other's VALU and
// LDS phases) where the LDS holds eight waves' tiles beside the codebook (64-dim values) and two
// waves' registers fit a SIMD; 4 for 128-dim values and for the variants that keep the most
// registers per tile (16 rows, or passthrough values loaded one by one together with a mask),
// which spill at 256 registers (16 rows without a mask at 8 waves: 30.0 µs against 28.1 µs at 4,
// B16 · 32/2 heads · T8192).
__host__ __device__ constexpr int contig_waves(int dt, int hv, bool mk, int r4) {
    return dt > 4 || r4 == 4 || (hv == 1 && mk) ? 4 : 8;
}

template <int BD, int DT, int VT, bool HAS_V, int HV, bool MK, int PB, int R4>
__global__ __launch_bounds__(contig_waves(DT, HV, MK, R4) * SSQ_WAVE) void k_decode_contig(const SsqContigParams p) {
    constexpr int NB = kD / BD;
    constexpr int RP = 4 * R4;  // query rows, padded to whole row quads
    constexpr int KR = kD / 16;  // A registers per row quad
    constexpr int Dv = 16 * DT;
    extern __shared__ __align__(16) float smem[];
    const ssq_decode_args& a = p.a;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar loop control
    constexpr int W = contig_waves(DT, HV, MK, R4);             // waves in the workgroup (the launch's)
    const int l16 = lane & 15, lg = lane >> 4;
    const int bk = blockIdx.x;
    const int split = blockIdx.y;
    const int b = bk / a.num_kv_heads;
    const int kv = bk - b * a.num_kv_heads;
    const int nc = a.n_centroids;
    const int nr = p.rows;
    const int t_begin = split * p.split_len;
    const int t_end = min(a.seq_len, t_begin + p.split_len);

    float* cb = smem;  // codebook [NB][nc][BD] fp32
    uint8_t* wreg = reinterpret_cast<uint8_t*>(smem + cb_floats(nc)) + wave * wave_bytes(DT);
    uint16_t* vt = reinterpret_cast<uint16_t*>(wreg);                     // [64][Dv]
    uint16_t* ps = reinterpret_cast<uint16_t*>(wreg + wave_v_bytes(DT));  // [16][64]

    // ---- prologue.  Issue order: this lane's permutation entries, the query rows unpermuted (lane j
    // loads dim j of each row, so no load waits for the permutation), the codebook through registers
    // (up to 8 float4s per thread per round, one round at 8 waves, two at 4), and the first two
    // tiles (each wave keeps two in flight).  Every load is a plain one: the compiler's waits for the
    // rows and the codebook then leave the tiles in flight (with a direct-to-LDS load pending it
    // would wait for all of them).  The scaled rows go through the wave's V-tile region (free until
    // the first tile) to be permuted into the A operand.
    const int jd = lane >> 2, iq = lane & 3;  // A-operand lane role: dim 16kk + jd of row 4q + iq
    const int64_t* perm = a.perm + (int64_t)kv * a.perm_sh;
    int64_t pj[KR];
#pragma unroll
    for (int kk = 0; kk < KR; ++kk) pj[kk] = perm[16 * kk + jd];
    const int64_t pjh = HV != 0 ? perm[p.hdim[jd]] : 0;  // hdim is 0 past n_hd

    uint32_t qlo[RP], qhi[RP];
    {
        int64_t src[RP];
#pragma unroll
        for (int r = 0; r < RP; ++r) {
            src[r] = lane;  // rows past nr read row 0 and are zeroed
            if (r < nr) {
                const int g = r / a.q_len, qi = r - g * a.q_len;
                const int h = kv * p.G + g;
                src[r] += (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)qi * a.q_sl;
            }
        }
        load_halves(a.q, a.q_dtype, src, qlo, qhi);
    }

    // codebook: float4 i of [NB][nc][BD] (16 nc of them) by thread i % (64 W); indices past the end
    // re-read (and re-store) the last one
    constexpr int kCbPer = 8;
    constexpr int kCbRounds = (16 * 256 + 64 * W * kCbPer - 1) / (64 * W * kCbPer);
    const v4u* cent4 = reinterpret_cast<const v4u*>(a.cent + (int64_t)kv * a.cent_sh);
    const int n4 = 16 * nc;
    v4u cbr[kCbPer];
    cb_load<kCbPer, W>(cent4, n4, tid, 0, cbr);

    const int n_tiles = (t_end - t_begin + kTile - 1) / kTile;
    const int last_tile = n_tiles > 0 ? n_tiles - 1 : 0;
    Tile<NB, DT, HV, MK, PB, RP> ra, rb;
    const int ta = t_begin + min(wave, last_tile) * kTile, tb = t_begin + min(wave + W, last_tile) * kTile;
    if constexpr (HAS_V) issue_values(p, b, kv, ta, t_end, lane, ra);
    issue_codes(p, b, kv, ta, t_end, lane, ra);
    cb_store<kCbPer, W>(cb, n4, tid, 0, cbr);
    if constexpr (kCbRounds > 1) {
        static_assert(kCbRounds == 2, "codebook rounds");
        if (64 * W * kCbPer < n4) {  // wave-uniform
            cb_load<kCbPer, W>(cent4, n4, tid, 1, cbr);
            if constexpr (HAS_V) issue_values(p, b, kv, tb, t_end, lane, rb);
            issue_codes(p, b, kv, tb, t_end, lane, rb);
            cb_store<kCbPer, W>(cb, n4, tid, 1, cbr);
        } else {
            if constexpr (HAS_V) issue_values(p, b, kv, tb, t_end, lane, rb);
            issue_codes(p, b, kv, tb, t_end, lane, rb);
        }
    } else {
        if constexpr (HAS_V) issue_values(p, b, kv, tb, t_end, lane, rb);
        issue_codes(p, b, kv, tb, t_end, lane, rb);
    }

    float qa[R4][KR];
    float qh[R4];
    {
        float* qs = reinterpret_cast<float*>(vt);  // [RP][64] scaled query rows, head dims unpermuted
#pragma unroll
        for (int r = 0; r < RP; ++r) {
            const float x = halves_to_f32(qlo[r], qhi[r], a.q_dtype);
            qs[r * kD + lane] = r >= nr ? 0.f : a.has_scale ? round_to_sel(x * a.scale, a.q_dtype) : x;
        }
        wave_sync();
#pragma unroll
        for (int q = 0; q < R4; ++q) {
            const float* qrow = qs + (4 * q + iq) * kD;
#pragma unroll
            for (int kk = 0; kk < KR; ++kk) {
                float x = qrow[min((uint64_t)pj[kk], (uint64_t)(kD - 1))];
                // passthrough blocks contribute through their stored values, not the codebook
                if (HV != 0 && ((a.heavy_mask[0] >> ((16 * kk + jd) / BD)) & 1ull)) x = 0.f;
                qa[q][kk] = x;
            }
            qh[q] = HV != 0 && jd < p.n_hd ? qrow[min((uint64_t)pjh, (uint64_t)(kD - 1))] : 0.f;
        }
        wave_sync();  // the rows are in registers: the region is the V tile's again
    }
    __syncthreads();  // every wave's share of the codebook is in LDS

    float m_run[RP], l_lane[RP];
    v4f acc[DT];
#pragma unroll
    for (int r = 0; r < RP; ++r) { m_run[r] = -INFINITY; l_lane[r] = 0.f; }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = (v4f){0.f, 0.f, 0.f, 0.f};

    // one tile: its values -> the wave's LDS region (and reloaded two rounds ahead), scores from the
    // registers, the rest reloaded, then softmax and P.V
    auto step = [&](Tile<NB, DT, HV, MK, PB, RP>& R, int tile) {
        const int t0 = t_begin + tile * kTile;
        const int t_next = t_begin + min(tile + 2 * W, last_tile) * kTile;
        if constexpr (HAS_V) {
            wave_sync();  // the previous tile's transposed reads of the region are done
#pragma unroll
            for (int i = 0; i < 2 * DT; ++i) *reinterpret_cast<uint4*>(vt + (i * SSQ_WAVE + lane) * 8) = R.v[i];
            issue_values(p, b, kv, t_next, t_end, lane, R);
        }
        float s[RP];
        tile_scores<BD, R4>(cb, nc, R, qa, qh, p.n_hd, a.pt_dtype, p.pk, s);
        if constexpr (MK) {
#pragma unroll
            for (int r = 0; r < RP; ++r) s[r] += R.mk[r];
        }
        issue_codes(p, b, kv, t_next, t_end, lane, R);

        const int t = t0 + lane;
        const bool valid = t < t_end;
        if (a.scores && valid) {
#pragma unroll
            for (int r = 0; r < RP; ++r) {
                if (r < nr) {
                    const int gq = r / a.q_len, qi = r - gq * a.q_len;
                    const int h = kv * p.G + gq;
                    a.scores[(int64_t)b * a.s_sb + (int64_t)h * a.s_sh + (int64_t)qi * a.s_sl + t] = s[r];
                }
            }
        }
        if constexpr (!HAS_V) return;

        // ---- online softmax per row over the wave's 64 tokens.  The running maximum m_run[r] is
        // wave-uniform and moves only when some score of the tile exceeds it by more than
        // kSoftmaxSlack, so most tiles skip the cross-lane maxima and the accumulator rescale.
        // Rows past nr come from zero query rows and are never stored.
        float sv[RP];
        bool over = false;
#pragma unroll
        for (int r = 0; r < RP; ++r) {
            sv[r] = valid ? s[r] : -INFINITY;
            over |= sv[r] > m_run[r] + kSoftmaxSlack;
        }
        if (__builtin_amdgcn_ballot_w64(over) != 0) {  // wave-uniform
            float alpha[RP];
#pragma unroll
            for (int r = 0; r < RP; ++r) {
                const float mn = fmaxf(m_run[r], wave_max64(sv[r]));
                alpha[r] = mn == -INFINITY ? 1.f : __expf(m_run[r] - mn);
                l_lane[r] *= alpha[r];
                m_run[r] = mn;
            }
            // accumulator row 4 g + i lives in lane group g = lane / 16
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float f = 1.f;
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    if (4 * g + i < RP) f = lg == g ? alpha[4 * g + i] : f;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) acc[dt][i] *= f;
            }
        }
#pragma unroll
        for (int r = 0; r < RP; ++r) {
            // m_run is -inf only while every score seen is -inf (then p = exp(-inf) = 0)
            const float mr = m_run[r] == -INFINITY ? 0.f : m_run[r];
            const float pr = __expf(sv[r] - mr);
            l_lane[r] += pr;
            ps[r * kTile + lane] = (uint16_t)to_vt16<VT>(pr);
        }
        wave_sync();

        // ---- P.V
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
            uint4 af = make_uint4(0, 0, 0, 0);
            if (l16 < RP) af = *reinterpret_cast<const uint4*>(ps + l16 * kTile + 32 * kh + 8 * lg);
            const int tr_tok = 32 * kh + 8 * lg + (l16 >> 2);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const uint16_t* src = vt + tr_tok * Dv + 16 * dt + 4 * (l16 & 3);
                const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) v4s*)(src));
                const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) v4s*)(src + 4 * Dv));
                const uint2 l2 = __builtin_bit_cast(uint2, lo);
                const uint2 h2 = __builtin_bit_cast(uint2, hi);
                acc[dt] = mfma_pv<VT>(af, make_uint4(l2.x, l2.y, h2.x, h2.y), acc[dt]);
            }
        }
    };
    // Two steps per trip and a single exit: a break between the steps made the compiler's
    // load-counter waits at the loop head drain both register sets, i.e. no tile ahead stayed in
    // flight.  A step past the last tile is harmless: its tokens are all past t_end, so they get
    // probability 0 and no score or mask access.
    for (int tile = wave; tile < n_tiles; tile += 2 * W) {
        step(ra, tile);
        step(rb, tile + W);
    }
    if constexpr (!HAS_V) return;

    // ---- merge the waves' (m, l, O) through LDS (the codebook is no longer needed)
    float l_w[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) l_w[r] = r < nr ? wave_sum64(l_lane[r]) : 0.f;
    __syncthreads();
    float* mbuf = smem;           // [waves][16]
    float* lbuf = mbuf + W * 16;  // [waves][16]
    float* obuf = lbuf + W * 16;  // [waves][16][Dv]
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RP; ++r) { mbuf[wave * 16 + r] = m_run[r]; lbuf[wave * 16 + r] = l_w[r]; }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (4 * lg + i < RP) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) obuf[((size_t)wave * 16 + 4 * lg + i) * Dv + 16 * dt + l16] = acc[dt][i];
        }
    __syncthreads();
    const int n_rows_all = a.batch * a.num_q_heads * a.q_len;
    for (int e = tid; e < nr * Dv; e += blockDim.x) {
        const int r = e / Dv, dv = e - r * Dv;
        float M = -INFINITY;
        for (int w = 0; w < W; ++w) M = fmaxf(M, mbuf[w * 16 + r]);
        float L = 0.f, o = 0.f;
        for (int w = 0; w < W; ++w) {
            const float mw = mbuf[w * 16 + r];
            if (mw == -INFINITY) continue;
            const float f = __expf(mw - M);
            L += lbuf[w * 16 + r] * f;
            o += obuf[((size_t)w * 16 + r) * Dv + dv] * f;
        }
        const int gq = r / a.q_len, qi = r - gq * a.q_len;
        const int h = kv * p.G + gq;
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

template <int BD, int DT, int VT, bool HAS_V, int HV, bool MK, int PB, int R4>
int launch_contig(const SsqContigParams& cp, const SsqContigPlan& pl, hipStream_t st) {
    auto kern = k_decode_contig<BD, DT, VT, HAS_V, HV, MK, PB, R4>;
    int rc = ssq_allow_lds((const void*)kern, (int)kMaxSmem, "hipFuncSetAttribute(decode_contig)");
    if (rc) return rc;
    constexpr int kW = contig_waves(DT, HV, MK, R4);
    SSQ_REQUIRE(pl.waves == kW, "decode_contig: %d waves planned, the variant runs %d", pl.waves, kW);
    dim3 grid(cp.a.batch * cp.a.num_kv_heads, pl.n_splits);
    hipLaunchKernelGGL(kern, grid, dim3(pl.waves * SSQ_WAVE), pl.smem, st, cp);
    return ssq_check_hip(hipGetLastError(), "k_decode_contig launch");
}

template <int DT, int VT, bool HAS_V, int HV, bool MK, int PB, int R4>
int contig_bd(const SsqContigParams& cp, const SsqContigPlan& pl, hipStream_t st) {
    switch (cp.a.block_dim) {
        case 1: return launch_contig<1, DT, VT, HAS_V, HV, MK, PB, R4>(cp, pl, st);
        case 2: return launch_contig<2, DT, VT, HAS_V, HV, MK, PB, R4>(cp, pl, st);
        case 4: return launch_contig<4, DT, VT, HAS_V, HV, MK, PB, R4>(cp, pl, st);
        default: return launch_contig<8, DT, VT, HAS_V, HV, MK, PB, R4>(cp, pl, st);
    }
}
template <int DT, int VT, bool HAS_V, int HV, bool MK, int PB>
int contig_r4(const SsqContigParams& cp, const SsqContigPlan& pl, hipStream_t st) {
    switch (pl.r4) {
        case 1: return contig_bd<DT, VT, HAS_V, HV, MK, PB, 1>(cp, pl, st);
        case 2: return contig_bd<DT, VT, HAS_V, HV, MK, PB, 2>(cp, pl, st);
        default: return contig_bd<DT, VT, HAS_V, HV, MK, PB, 4>(cp, pl, st);
    }
}
// the variants without passthrough values: byte codes with or without a mask, 4- and 6-bit words,
// other widths below 8 bits (taken at run time)
template <int DT, int VT, bool HAS_V>
int contig_plain(const SsqContigParams& cp, const SsqContigPlan& pl, hipStream_t st) {
    if (cp.a.code_bits == 4) return contig_r4<DT, VT, HAS_V, 0, false, 4>(cp, pl, st);
    if (cp.a.code_bits == 6) return contig_r4<DT, VT, HAS_V, 0, false, 6>(cp, pl, st);
    if (cp.a.code_bits > 0) return contig_r4<DT, VT, HAS_V, 0, false, -1>(cp, pl, st);  // 1-3, 5, 7 bits
    if (HAS_V && cp.a.mask) return contig_r4<DT, VT, HAS_V, 0, HAS_V, 0>(cp, pl, st);
    return contig_r4<DT, VT, HAS_V, 0, false, 0>(cp, pl, st);
}
// the passthrough (SunShape-Mixed) variants: one 16-byte load of 8 values, or one load per value
// with or without a mask
template <int DT, int VT, bool HAS_V>
int contig_mixed(const SsqContigParams& cp, const SsqContigPlan& pl, hipStream_t st) {
    if (cp.pt_vec && !cp.a.mask) return contig_r4<DT, VT, HAS_V, 2, false, 0>(cp, pl, st);
    if (HAS_V && cp.a.mask) return contig_r4<DT, VT, HAS_V, 1, HAS_V, 0>(cp, pl, st);
    return contig_r4<DT, VT, HAS_V, 1, false, 0>(cp, pl, st);
}

}  // namespace

// the instantiation units (ssq_decode_contig_<values>_<variants>.hip)
#define SSQ_CONTIG_UNIT(name) int name(const SsqContigParams& cp, const SsqContigPlan& pl, hipStream_t st)
SSQ_CONTIG_UNIT(ssq_contig_scores_plain);
SSQ_CONTIG_UNIT(ssq_contig_scores_mixed);
SSQ_CONTIG_UNIT(ssq_contig_64_bf16_plain);
SSQ_CONTIG_UNIT(ssq_contig_64_bf16_mixed);
SSQ_CONTIG_UNIT(ssq_contig_64_f16_plain);
SSQ_CONTIG_UNIT(ssq_contig_64_f16_mixed);
SSQ_CONTIG_UNIT(ssq_contig_128_bf16_plain);
SSQ_CONTIG_UNIT(ssq_contig_128_bf16_mixed);
SSQ_CONTIG_UNIT(ssq_contig_128_f16_plain);
SSQ_CONTIG_UNIT(ssq_contig_128_f16_mixed);
