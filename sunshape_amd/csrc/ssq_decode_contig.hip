// Fused VQ-key decode (and scores) over the reference's contiguous layout on the matrix cores.
//
// Same mathematics as the other decode kernels (q scaled in its own dtype, softmax in fp32, the
// probabilities cast to the value dtype before P.V: vllm_attn_backend.py:232-252), mapped for
// contiguous token-major values [B, Hkv, T, Dv] and head_dim 64:
//
//   scores = v_mfma_f32_16x16x4f32 over Qp [16 rows x 64] . K_hat^T: the permuted, scaled query
//            rows are a fixed A operand held in registers; each lane gathers its B element
//            K_hat[token][dim] = C[blk][code][d] from the codebook staged in LDS.  No LUT is built,
//            so up to 16 query rows share one pass over the keys.  fp32 products and sums; the
//            order differs from the LUT kernels' (block by block), within fp32 rounding.
//   P.V    = v_mfma_f32_16x16x32_bf16 (_f16): A = P [16 rows x 32 tokens] from a per-wave LDS strip;
//            B = V [32 tokens x 16 dims].  V tiles are copied to LDS with coalesced 16-byte loads
//            and read back transposed with ds_read_b64_tr_b16: within each 16-lane group, lane l
//            addresses V[t0 + l/4][n0 + 4*(l%4) .. +3] and receives V[t0 .. t0+3][n0 + l], so two
//            reads give a lane its 8 consecutive tokens of one dim.
//
// Codes arrive as byte rows or as 4- / 6-bit codes packed into int32 words
// (sunshape/triton_kernels.py:250-266); packed rows are loaded as words and unpacked to bytes when
// the tile is copied to LDS, so the score loop is the same for both.
//
// workgroup = 4 waves for one (batch, KV head, context split); each wave streams 64-token tiles with
// its own running (max, sum, O), the next tile's loads in flight; waves merge through LDS at the end.
#include "ssq_common.h"

#include <math.h>

int ssq_launch_merge(const ssq_decode_args& a, int n_splits, const float* ws_o, const float* ws_m,
                     const float* ws_l, hipStream_t st);

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr int kMaxWaves = 8;  // waves per workgroup: 8 where the LDS and registers allow, else 4
constexpr int kTile = 64;  // tokens per wave iteration
constexpr int kD = 64;     // head_dim served
constexpr int kHP = 16;    // passthrough (heavy-block) dims per token, padded to whole MFMA steps
constexpr size_t kMaxSmem = 160 * 1024;

struct ContigParams {
    ssq_decode_args a;
    int G, rows, split_len, n_splits;
    float* ws_o;
    float* ws_m;
    float* ws_l;
    // passthrough dims (SunShape-Mixed): the token record element and the permuted head dim of
    // heavy dim idx (blocks ascending, then d); n_hd of them
    int n_hd;
    int pt_vec;  // 1: the 8 passthrough values are contiguous 16-bit elements from slot 0, 16-byte aligned
    int hoff[kHP];
    int hdim[kHP];
};

// per-wave LDS region (bytes): V tile [64][Dv] (16-bit) | codes [64][NB] | P strip [16][64] (16-bit)
//                               | passthrough values [64][kHP] fp32 (heavy blocks only)
__host__ __device__ constexpr int wave_v_bytes(int DT) { return kTile * DT * 16 * 2; }
__host__ __device__ constexpr int wave_bytes(int NB, int DT, bool HV) {
    return wave_v_bytes(DT) + kTile * NB + 16 * kTile * 2 + (HV ? kTile * kHP * 4 : 0);
}
// codebook region: [NB][nc][BD] fp32, padded to whole 1 KB chunks (one direct-to-LDS wave load each)
__host__ __device__ constexpr int cb_floats(int nc) { return (16 * nc + 63) / 64 * 256; }
inline size_t contig_smem(const ssq_decode_args& a, int DT, int waves) {
    const bool hv = (a.heavy_mask[0] | a.heavy_mask[1]) != 0;
    const size_t cb = (size_t)cb_floats(a.n_centroids) * 4;
    const size_t main = cb + (size_t)waves * wave_bytes(a.n_blocks, DT, hv);
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
// max / sum over the 16 lanes of a row (every lane of the row receives the result)
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dpp_ror<0x121>(v)); v = fmaxf(v, dpp_ror<0x122>(v));
    v = fmaxf(v, dpp_ror<0x124>(v)); v = fmaxf(v, dpp_ror<0x128>(v));
    return v;
}
__device__ __forceinline__ float row_sum(float v) {
    v += dpp_ror<0x121>(v); v += dpp_ror<0x122>(v);
    v += dpp_ror<0x124>(v); v += dpp_ror<0x128>(v);
    return v;
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// packed code rows (PB bits per code, 32 / PB codes per little-endian int32 word, the low bits
// first; sunshape/triton_kernels.py:250-266): int32 words per row
__host__ __device__ constexpr int pk_words(int NB, int PB) { return PB ? (NB + 32 / PB - 1) / (32 / PB) : 1; }

// registers of one 64-token tile in flight: this lane's 16-byte V chunks, its token's code row
// (bytes, or PB-bit codes in words) and (heavy blocks) its token's passthrough values
// HV: passthrough values per token: 0 none; 1 up to kHP values, one load each (any dtype and
// slot layout); 2 exactly 8 contiguous 16-bit values from slot 0, one 16-byte load
template <int NB, int DT, int HV, bool MK, int PB>
struct Tile {
    uint4 v[2 * DT];
    uint4 c[NB >= 16 ? NB / 16 : 1];
    uint2 c8;
    uint32_t pk[pk_words(NB, PB)];
    uint32_t h[HV == 1 ? kHP : HV == 2 ? 4 : 1];  // raw bits; converted when the tile goes to LDS
    float mk[MK ? 16 : 1];     // additive mask at [row 4*lg + i][token 16g + l16], index 4g + i
};

// Loads are unconditional; chunks of tokens past the split's end re-read the last token's row
// (valid memory; such tokens get p = 0 and are never scored).
template <int NB, int DT, bool HAS_V, int HV, bool MK, int PB>
__device__ __forceinline__ void issue_tile(const ContigParams& p, int b, int kv, int t0, int t_end, int lane,
                                           Tile<NB, DT, HV, MK, PB>& R) {
    const ssq_decode_args& a = p.a;
    const int tc = min(t0 + lane, t_end - 1);
    if constexpr (MK) {  // clamped offsets; entries of invalid (row, token) pairs are never added
        const int l16 = lane & 15, lg = lane >> 4;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int t = min(t0 + 16 * g + l16, t_end - 1);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = min(4 * lg + i, p.rows - 1);
                const int gq = r / a.q_len, qi = r - gq * a.q_len;
                const int h = kv * p.G + gq;
                R.mk[4 * g + i] =
                    a.mask[(int64_t)b * a.m_sb + (int64_t)h * a.m_sh + (int64_t)qi * a.m_sl + (int64_t)t * a.m_st];
            }
        }
    }
    if constexpr (HV == 1) {
        const int64_t pb = (int64_t)b * a.pt_sb + (int64_t)kv * a.pt_sh + (int64_t)tc * a.pt_st;
#pragma unroll
        for (int i = 0; i < kHP; ++i) R.h[i] = ssq_load_bits(a.pt, a.pt_dtype, pb + p.hoff[i]);  // hoff clamped
    } else if constexpr (HV == 2) {
        const int64_t pb = (int64_t)b * a.pt_sb + (int64_t)kv * a.pt_sh + (int64_t)tc * a.pt_st;
        const uint4 w = ld16(reinterpret_cast<const uint16_t*>(a.pt) + pb);
        R.h[0] = w.x; R.h[1] = w.y; R.h[2] = w.z; R.h[3] = w.w;
    }
    if constexpr (PB) {  // packed rows: strides count int32 words
        const uint32_t* prow = reinterpret_cast<const uint32_t*>(a.codes) + (int64_t)b * a.c_sb +
                               (int64_t)kv * a.c_sh + (int64_t)tc * a.c_st;
#pragma unroll
        for (int i = 0; i < pk_words(NB, PB); ++i) R.pk[i] = __builtin_nontemporal_load(prow + i);
    } else if constexpr (NB >= 16) {
        const uint8_t* crow = a.codes + (int64_t)b * a.c_sb + (int64_t)kv * a.c_sh + (int64_t)tc * a.c_st;
#pragma unroll
        for (int i = 0; i < NB / 16; ++i) R.c[i] = ld16(crow + 16 * i);
    } else {
        const uint8_t* crow = a.codes + (int64_t)b * a.c_sb + (int64_t)kv * a.c_sh + (int64_t)tc * a.c_st;
        R.c8 = *reinterpret_cast<const uint2*>(crow);
    }
    if constexpr (HAS_V) {
        const uint16_t* vb = reinterpret_cast<const uint16_t*>(a.v) + (int64_t)b * a.v_sb + (int64_t)kv * a.v_sh;
        constexpr int kRowChunks = 2 * DT;  // 16-byte chunks per token row (Dv = 16 * DT)
#pragma unroll
        for (int i = 0; i < 2 * DT; ++i) {
            const int chunk = i * SSQ_WAVE + lane;  // chunk of the tile, row-major
            const int tok = min(t0 + chunk / kRowChunks, t_end - 1);
            R.v[i] = ld16(vb + (int64_t)tok * a.v_st + (chunk % kRowChunks) * 8);
        }
    }
}

// Waves per workgroup.  8 need two waves' registers per SIMD, which the variants without
// passthrough, mask or 128-dim values fit; the others keep 4.  (The passthrough variants' tiles
// leave LDS for only 6 waves beside a 64 KiB codebook; 6 waves put two on only two of the four
// SIMDs and measured slower than 4.)
__host__ __device__ constexpr int contig_waves(int dt, int hv, bool mk) { return !mk && dt <= 4 && hv == 0 ? 8 : 4; }

template <int BD, int DT, int VT, bool HAS_V, int HV, bool MK, int PB>
__global__ __launch_bounds__(contig_waves(DT, HV, MK) * SSQ_WAVE) void k_decode_contig(
    const ContigParams p) {
    constexpr int NB = kD / BD;
    constexpr int NBW = NB / 4;  // code row dwords
    constexpr int KS = kD / 4;   // score k-steps
    constexpr int Dv = 16 * DT;
    extern __shared__ __align__(16) float smem[];
    const ssq_decode_args& a = p.a;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar loop control
    const int W = blockDim.x >> 6;                              // waves in the workgroup
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
    uint8_t* wreg = reinterpret_cast<uint8_t*>(smem + cb_floats(nc)) + wave * wave_bytes(NB, DT, HV != 0);
    uint16_t* vt = reinterpret_cast<uint16_t*>(wreg);                            // [64][Dv]
    uint8_t* ct = wreg + wave_v_bytes(DT);                                       // [64][NB]
    uint16_t* ps = reinterpret_cast<uint16_t*>(wreg + wave_v_bytes(DT) + kTile * NB);  // [16][64]
    float* ph = reinterpret_cast<float*>(wreg + wave_v_bytes(DT) + kTile * NB + 16 * kTile * 2);  // [64][kHP]

    // ---- prologue.  Issue order: this lane's permutation entries, the first two tiles (two register
    // sets in flight: a set is free again once its tile is in LDS, and then loads the tile two rounds
    // ahead), the codebook, and the query rows unpermuted (lane j loads dim j of each row, so no load
    // waits for the permutation): one memory latency in all.  The scaled rows then go through the
    // wave's V-tile region (free until the first tile) to be permuted into the A operand.
    const int64_t* perm = a.perm + (int64_t)kv * a.perm_sh;
    int64_t pj[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) pj[s] = perm[4 * s + lg];
    int64_t pjh[HV != 0 ? kHP / 4 : 1];  // passthrough pass: permuted head dim of heavy dim 4s + lg
    if constexpr (HV != 0) {
#pragma unroll
        for (int s = 0; s < kHP / 4; ++s) pjh[s] = perm[p.hdim[4 * s + lg]];  // hdim is 0 past n_hd
    }

    const int n_tiles = (t_end - t_begin + kTile - 1) / kTile;
    const int last_tile = n_tiles > 0 ? n_tiles - 1 : 0;
    Tile<NB, DT, HV, MK, PB> ra, rb;
    if (n_tiles > 0) {
        issue_tile<NB, DT, HAS_V, HV, MK, PB>(p, b, kv, t_begin + min(wave, last_tile) * kTile, t_end, lane, ra);
        issue_tile<NB, DT, HAS_V, HV, MK, PB>(p, b, kv, t_begin + min(wave + W, last_tile) * kTile, t_end, lane, rb);
    }

    // the codebook goes global -> LDS directly (no registers): 1 KB chunks, lane l's 16 bytes at
    // chunk + 16 l; the tail chunk's lanes past the end re-read the last float4 into the padding
    {
        const float* cent = a.cent + (int64_t)kv * a.cent_sh;
        const int n4 = 16 * nc;  // float4s: NB * nc * BD = 64 nc floats
        const int n_chunks = (n4 + 63) / 64;
        for (int c = wave; c < n_chunks; c += W) {
            const int i = min(c * 64 + lane, n4 - 1);
            __builtin_amdgcn_global_load_lds(cent + 4 * i, (__attribute__((address_space(3))) void*)(cb + 256 * c), 16, 0,
                                             0);
        }
    }

    float qa[KS];
    float qh[HV != 0 ? kHP / 4 : 1];  // A operand of the passthrough pass: Qp[row l16][heavy dim 4s + lg]
    {
        constexpr int kRows = 16;  // A-operand rows (nr <= 16)
        int64_t src[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            src[r] = lane;  // rows past nr read row 0 and are zeroed
            if (r < nr) {
                const int g = r / a.q_len, qi = r - g * a.q_len;
                const int h = kv * p.G + g;
                src[r] += (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)qi * a.q_sl;
            }
        }
        float qv[kRows];
        ssq_load_elems(a.q, a.q_dtype, src, qv);
        float* qs = reinterpret_cast<float*>(vt);  // [16][64] scaled query rows, head dims unpermuted
#pragma unroll
        for (int r = 0; r < kRows; ++r)
            qs[r * kD + lane] = r >= nr ? 0.f : a.has_scale ? ssq_round_to(qv[r] * a.scale, a.q_dtype) : qv[r];
        wave_sync();
        const float* qrow = qs + l16 * kD;
#pragma unroll
        for (int s = 0; s < KS; ++s) qa[s] = qrow[min((uint64_t)pj[s], (uint64_t)(kD - 1))];
        if constexpr (HV != 0) {
#pragma unroll
            for (int s = 0; s < kHP / 4; ++s)  // heavy dims past n_hd are zero
                qh[s] = 4 * s + lg < p.n_hd ? qrow[min((uint64_t)pjh[s], (uint64_t)(kD - 1))] : 0.f;
            // passthrough blocks contribute through their stored values (second pass), not the codebook
#pragma unroll
            for (int s = 0; s < KS; ++s)
                if ((a.heavy_mask[0] >> ((4 * s + lg) / BD)) & 1ull) qa[s] = 0.f;
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's direct-to-LDS codebook loads have landed
    __syncthreads();

    // Codebook gather of step s: this lane supplies head dim j = 4s + lg, i.e. dim j % BD of block
    // j / BD.  For BD in {1, 2, 4, 8} the block's LDS byte offset and its code's bit position in the
    // step's code word split into a per-step (uniform) part and a per-lane part, so no per-step
    // tables are kept:  offset = lane_off + step_off(s) + code * BD * 4,  bit = lane_sh + step_sh(s).
    constexpr int kLogBD = BD == 1 ? 0 : BD == 2 ? 1 : BD == 4 ? 2 : 3;
    const uint8_t* cbb = reinterpret_cast<const uint8_t*>(cb);
    const uint32_t ncm1 = (uint32_t)(nc - 1);
    const uint32_t lane_off = BD <= 4 ? (uint32_t)(((lg >> kLogBD) * nc * BD) + (lg & (BD - 1))) * 4u : 4u * lg;
    const uint32_t lane_sh = BD == 1 ? 8u * lg : BD == 2 ? 8u * (lg >> 1) : 0u;
    float m_run[4], l_run[4];
    v4f acc[DT];
#pragma unroll
    for (int i = 0; i < 4; ++i) { m_run[i] = -INFINITY; l_run[i] = 0.f; }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = (v4f){0.f, 0.f, 0.f, 0.f};

    // one tile: its registers -> the wave's LDS region, the set reloaded two rounds ahead, compute
    auto step = [&](Tile<NB, DT, HV, MK, PB>& R, int tile) {
        const int t0 = t_begin + tile * kTile;
        wave_sync();
        if constexpr (PB) {  // unpack to one byte per code: the score loop reads byte rows either way
            constexpr int kVpe = 32 / PB;
            constexpr uint32_t kMsk = (1u << PB) - 1u;
            uint32_t u[NB / 4];
#pragma unroll
            for (int j = 0; j < NB / 4; ++j) u[j] = 0u;
#pragma unroll
            for (int i = 0; i < NB; ++i) u[i >> 2] |= ((R.pk[i / kVpe] >> ((i % kVpe) * PB)) & kMsk) << (8 * (i & 3));
            if constexpr (NB >= 16) {
#pragma unroll
                for (int i = 0; i < NB / 16; ++i)
                    *reinterpret_cast<uint4*>(ct + lane * NB + 16 * i) =
                        make_uint4(u[4 * i], u[4 * i + 1], u[4 * i + 2], u[4 * i + 3]);
            } else {
                *reinterpret_cast<uint2*>(ct + lane * NB) = make_uint2(u[0], u[1]);
            }
        } else if constexpr (NB >= 16) {
#pragma unroll
            for (int i = 0; i < NB / 16; ++i) *reinterpret_cast<uint4*>(ct + lane * NB + 16 * i) = R.c[i];
        } else {
            *reinterpret_cast<uint2*>(ct + lane * NB) = R.c8;
        }
        if constexpr (HAS_V) {
#pragma unroll
            for (int i = 0; i < 2 * DT; ++i) *reinterpret_cast<uint4*>(vt + (i * SSQ_WAVE + lane) * 8) = R.v[i];
        }
        if constexpr (HV == 1) {
#pragma unroll
            for (int i = 0; i < kHP; i += 4) {
                float x[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) x[u] = i + u < p.n_hd ? ssq_bits_to_f32(R.h[i + u], a.pt_dtype) : 0.f;
                *reinterpret_cast<float4*>(ph + lane * kHP + i) = make_float4(x[0], x[1], x[2], x[3]);
            }
        } else if constexpr (HV == 2) {  // 8 values, two per word (low half first); dims 8..15 are zero
#pragma unroll
            for (int i = 0; i < 8; i += 4) {
                float x[4];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    x[u] = ssq_bits_to_f32((R.h[(i + u) >> 1] >> (16 * ((i + u) & 1))) & 0xFFFFu, a.pt_dtype);
                *reinterpret_cast<float4*>(ph + lane * kHP + i) = make_float4(x[0], x[1], x[2], x[3]);
            }
            *reinterpret_cast<float4*>(ph + lane * kHP + 8) = make_float4(0.f, 0.f, 0.f, 0.f);
            *reinterpret_cast<float4*>(ph + lane * kHP + 12) = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        wave_sync();
        float mk[MK ? 16 : 1];  // this tile's mask values, taken before R is reloaded
#pragma unroll
        for (int k = 0; k < (MK ? 16 : 1); ++k) mk[k] = MK ? R.mk[k] : 0.f;
        issue_tile<NB, DT, HAS_V, HV, MK, PB>(p, b, kv, t_begin + min(tile + 2 * W, last_tile) * kTile, t_end, lane, R);

        // ---- scores: S[row 4*lg+i][token 16g + l16] for the tile's 4 groups of 16 tokens
        v4f sc[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint32_t cw[NBW];
            const uint8_t* crow = ct + (16 * g + l16) * NB;
            if constexpr (NB >= 16) {
#pragma unroll
                for (int i = 0; i < NB / 16; ++i) {
                    const uint4 w = *reinterpret_cast<const uint4*>(crow + 16 * i);
                    cw[4 * i] = w.x; cw[4 * i + 1] = w.y; cw[4 * i + 2] = w.z; cw[4 * i + 3] = w.w;
                }
            } else {
                const uint2 w = *reinterpret_cast<const uint2*>(crow);
                cw[0] = w.x; cw[1] = w.y;
            }
            v4f c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                // the word holding this step's block code is the same for every lg (BD in {1,2,4,8})
                const uint32_t word = cw[((4 * s) / BD) >> 2];
                const uint32_t step_sh = BD == 1 ? 0u : BD == 2 ? 16u * (s & 1) : BD == 4 ? 8u * (s & 3) : 8u * ((s >> 1) & 3);
                const uint32_t step_off = BD <= 4 ? (uint32_t)s * 16u * (uint32_t)nc
                                                  : (uint32_t)(s >> 1) * 32u * (uint32_t)nc + 16u * (s & 1);
                const uint32_t code = min(__builtin_amdgcn_ubfe(word, lane_sh + step_sh, 8), ncm1);
                const float kval = *reinterpret_cast<const float*>(cbb + lane_off + step_off + (code << (2 + kLogBD)));
                c = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s], kval, c, 0, 0, 0);
            }
            if constexpr (HV != 0) {  // passthrough pass: B = the tokens' stored heavy-block values
#pragma unroll
                for (int s = 0; s < kHP / 4; ++s) {
                    if (4 * s < p.n_hd) {
                        const float kval = ph[(16 * g + l16) * kHP + 4 * s + lg];
                        c = __builtin_amdgcn_mfma_f32_16x16x4f32(qh[s], kval, c, 0, 0, 0);
                    }
                }
            }
            sc[g] = c;
        }
        // additive mask (loaded with the tile), raw-score output
        if constexpr (MK) {
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (4 * lg + i < nr && t0 + 16 * g + l16 < t_end) sc[g][i] += mk[4 * g + i];
        }
        if (a.scores) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int t = t0 + 16 * g + l16;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 4 * lg + i;
                    if (r < nr && t < t_end) {
                        const int gq = r / a.q_len, qi = r - gq * a.q_len;
                        const int h = kv * p.G + gq;
                        a.scores[(int64_t)b * a.s_sb + (int64_t)h * a.s_sh + (int64_t)qi * a.s_sl + t] = sc[g][i];
                    }
                }
            }
        }
        if constexpr (!HAS_V) return;

        // ---- online softmax (rows 4*lg + i live in this lane's row of 16 lanes)
        float alpha[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float mx = -INFINITY;
#pragma unroll
            for (int g = 0; g < 4; ++g)
                if (t0 + 16 * g + l16 < t_end) mx = fmaxf(mx, sc[g][i]);
            mx = row_max(mx);
            const float mn = fmaxf(m_run[i], mx);
            alpha[i] = (mn == -INFINITY) ? 1.f : __expf(m_run[i] - mn);
            m_run[i] = mn;
            float lsum = 0.f;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const bool valid = t0 + 16 * g + l16 < t_end;
                const float pr = (valid && mn != -INFINITY) ? __expf(sc[g][i] - mn) : 0.f;
                lsum += pr;
                ps[(4 * lg + i) * kTile + 16 * g + l16] = (uint16_t)to_vt16<VT>(pr);
            }
            l_run[i] = l_run[i] * alpha[i] + lsum;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) acc[dt][i] *= alpha[i];
        }
        wave_sync();

        // ---- P.V
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
            const uint4 af = *reinterpret_cast<const uint4*>(ps + l16 * kTile + 32 * kh + 8 * lg);
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
    float l_w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) l_w[i] = row_sum(l_run[i]);
    __syncthreads();
    float* mbuf = smem;               // [waves][16]
    float* lbuf = mbuf + W * 16;  // [waves][16]
    float* obuf = lbuf + W * 16;  // [waves][16][Dv]
    if (l16 == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) { mbuf[wave * 16 + 4 * lg + i] = m_run[i]; lbuf[wave * 16 + 4 * lg + i] = l_w[i]; }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) obuf[((size_t)wave * 16 + 4 * lg + i) * Dv + 16 * dt + l16] = acc[dt][i];
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

// passthrough dims of the heavy blocks, blocks ascending then d: the token record element and
// the permuted head dim of each (n_hd of them), and whether they are 8 contiguous 16-bit
// elements from slot 0 in 16-byte aligned rows (the one-load variant)
struct PtLayout {
    int n_hd = 0, vec = 0;
    int hoff[kHP] = {}, hdim[kHP] = {};
};
PtLayout pt_layout(const ssq_decode_args& a) {
    PtLayout L;
    for (int blk = 0, h = 0; blk < a.n_blocks && blk < 64; ++blk) {
        if (!((a.heavy_mask[0] >> blk) & 1ull)) continue;
        const int slot = a.pt_dense ? blk : h;  // record slot = block (dense) or ordinal
        for (int d = 0; d < a.block_dim && L.n_hd < kHP; ++d) {
            L.hoff[L.n_hd] = slot * a.block_dim + d;
            L.hdim[L.n_hd] = blk * a.block_dim + d;
            ++L.n_hd;
        }
        ++h;
    }
    for (int i = L.n_hd; i < kHP; ++i) L.hoff[i] = L.hoff[0];  // loaded, then zeroed in the kernel
    if (L.n_hd == 8 && (a.pt_dtype == SSQ_BF16 || a.pt_dtype == SSQ_F16) && (uintptr_t)a.pt % 16 == 0 &&
        (a.pt_sb * 2) % 16 == 0 && (a.pt_sh * 2) % 16 == 0 && (a.pt_st * 2) % 16 == 0) {
        L.vec = 1;
        for (int i = 0; i < 8; ++i) L.vec &= L.hoff[i] == i ? 1 : 0;
    }
    return L;
}
// the kernel's passthrough variant: 0 none, 1 one load per value, 2 one 16-byte load (no mask)
int hv_kind(const ssq_decode_args& a, const PtLayout& L) {
    return L.n_hd == 0 ? 0 : L.vec && !a.mask ? 2 : 1;
}

struct CPlan {
    int DT, split_len, n_splits, waves;
    size_t smem, ws_bytes;
};

bool plan(const ssq_decode_args* a, bool has_v, CPlan& pl) {
    if (a->layout != SSQ_CONTIGUOUS) return false;
    // packed codes: 4- and 6-bit words are unpacked in the kernel (without passthrough or mask);
    // 8-bit words are byte rows (strides scaled to bytes); other widths take the generic kernel
    const int cbits = a->code_bits;
    if (cbits != 0 && cbits != 4 && cbits != 6 && cbits != 8) return false;
    if ((cbits == 4 || cbits == 6) && (a->heavy_mask[0] || a->mask)) return false;
    if (a->heavy_mask[1]) return false;
    if (a->heavy_mask[0]) {
        const int n_hd = __builtin_popcountll(a->heavy_mask[0]) * a->block_dim;
        if (n_hd > kHP || !a->pt || a->pt_dtype < SSQ_F32 || a->pt_dtype > SSQ_F16) return false;
    }
    if (a->head_dim != kD) return false;
    const int bd = a->block_dim;
    if (bd != 1 && bd != 2 && bd != 4 && bd != 8) return false;
    if (a->n_centroids > 256) return false;
    const int rows = (a->num_q_heads / a->num_kv_heads) * a->q_len;
    if (rows > 16) return false;
    if ((uintptr_t)a->cent % 16 || (a->cent_sh * 4) % 16) return false;
    const int nb = a->n_blocks;
    if (cbits == 4 || cbits == 6) {  // word loads
        if ((uintptr_t)a->codes % 4) return false;
    } else {
        const int cal = nb >= 16 ? 16 : 8;  // code row loads of 16 (or 8) bytes
        const int64_t cs = cbits == 8 ? 4 : 1;  // stride unit in bytes
        if ((uintptr_t)a->codes % cal || (a->c_st * cs) % cal || (a->c_sh * cs) % cal || (a->c_sb * cs) % cal)
            return false;
    }
    pl.DT = 4;
    if (has_v) {
        if (a->v_dtype != SSQ_BF16 && a->v_dtype != SSQ_F16) return false;
        if (a->value_dim != 64 && a->value_dim != 128) return false;
        if ((uintptr_t)a->v % 16 || (a->v_sb * 2) % 16 || (a->v_sh * 2) % 16 || (a->v_st * 2) % 16) return false;
        pl.DT = a->value_dim / 16;
    }
    // 8 waves share the codebook where the LDS holds their tiles (two waves per SIMD hide each
    // other's gather and MFMA latency) and the registers allow; otherwise 4
    pl.waves = contig_waves(pl.DT, hv_kind(*a, pt_layout(*a)), a->mask != nullptr);
    if (contig_smem(*a, pl.DT, pl.waves) > kMaxSmem) pl.waves = 4;
    pl.smem = contig_smem(*a, pl.DT, pl.waves);
    if (pl.smem > kMaxSmem) return false;
    const int units = a->batch * a->num_kv_heads;
    const int tiles = (a->seq_len + kTile - 1) / kTile;
    const int cus = ssq_device_cus();
    int splits = a->num_splits > 0 ? a->num_splits : (cus + units - 1) / units;
    const int max_splits = (tiles + pl.waves - 1) / pl.waves;
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    const int tiles_per_split = (tiles + splits - 1) / splits;
    pl.split_len = tiles_per_split * kTile;
    pl.n_splits = (a->seq_len + pl.split_len - 1) / pl.split_len;
    if (pl.n_splits < 1) pl.n_splits = 1;
    const size_t n_rows_all = (size_t)a->batch * a->num_q_heads * a->q_len;
    pl.ws_bytes = (has_v && pl.n_splits > 1) ? (size_t)pl.n_splits * n_rows_all * (a->value_dim + 2) * 4 : 0;
    return true;
}

template <int BD, int DT, int VT, bool HAS_V, int HV, bool MK, int PB>
int launch(const ContigParams& cp, const CPlan& pl, hipStream_t st) {
    auto kern = k_decode_contig<BD, DT, VT, HAS_V, HV, MK, PB>;
    int rc = ssq_allow_lds((const void*)kern, (int)kMaxSmem, "hipFuncSetAttribute(decode_contig)");
    if (rc) return rc;
    dim3 grid(cp.a.batch * cp.a.num_kv_heads, pl.n_splits);
    SSQ_REQUIRE(pl.waves <= contig_waves(DT, HV, MK), "decode_contig: %d waves exceed the variant's %d", pl.waves,
                contig_waves(DT, HV, MK));
    hipLaunchKernelGGL(kern, grid, dim3(pl.waves * SSQ_WAVE), pl.smem, st, cp);
    return ssq_check_hip(hipGetLastError(), "k_decode_contig launch");
}

template <int DT, int VT, bool HAS_V, int HV, bool MK, int PB = 0>
int launch_bd(const ContigParams& cp, const CPlan& pl, hipStream_t st) {
    switch (cp.a.block_dim) {
        case 1: return launch<1, DT, VT, HAS_V, HV, MK, PB>(cp, pl, st);
        case 2: return launch<2, DT, VT, HAS_V, HV, MK, PB>(cp, pl, st);
        case 4: return launch<4, DT, VT, HAS_V, HV, MK, PB>(cp, pl, st);
        default: return launch<8, DT, VT, HAS_V, HV, MK, PB>(cp, pl, st);
    }
}
template <int DT, int VT, bool HAS_V, int HV>
int launch_mk(const ContigParams& cp, const CPlan& pl, hipStream_t st) {
    return cp.a.mask ? launch_bd<DT, VT, HAS_V, HV, true>(cp, pl, st) : launch_bd<DT, VT, HAS_V, HV, false>(cp, pl, st);
}
template <int DT, int VT, bool HAS_V>
int launch_hv(const ContigParams& cp, const CPlan& pl, hipStream_t st) {
    if (cp.a.code_bits == 4) return launch_bd<DT, VT, HAS_V, 0, false, 4>(cp, pl, st);
    if (cp.a.code_bits == 6) return launch_bd<DT, VT, HAS_V, 0, false, 6>(cp, pl, st);
    if (hv_kind(cp.a, PtLayout{cp.n_hd, cp.pt_vec}) == 2) return launch_bd<DT, VT, HAS_V, 2, false>(cp, pl, st);
    return cp.n_hd > 0 ? launch_mk<DT, VT, HAS_V, 1>(cp, pl, st) : launch_mk<DT, VT, HAS_V, 0>(cp, pl, st);
}

}  // namespace

int ssq_decode_contig_supported(const ssq_decode_args* a) {
    CPlan pl;
    return plan(a, a->v != nullptr, pl) ? 1 : 0;
}

size_t ssq_decode_contig_workspace(const ssq_decode_args* a) {
    CPlan pl;
    return plan(a, a->v != nullptr, pl) ? pl.ws_bytes : 0;
}

// decode (a->v != NULL) or scores only (a->v == NULL, a->scores != NULL)
int ssq_decode_contig(const ssq_decode_args* a, void* workspace, size_t ws_bytes, hipStream_t st) {
    const bool has_v = a->v != nullptr;
    CPlan pl;
    if (!plan(a, has_v, pl)) return ssq_fail(SSQ_ERR_UNSUPPORTED, "contiguous MFMA kernel does not support this problem");
    if (a->seq_len == 0) {
        if (!has_v) return SSQ_OK;
        return ssq_fail(SSQ_ERR_INVALID, "seq_len == 0: softmax over an empty context");
    }
    SSQ_REQUIRE(ws_bytes >= pl.ws_bytes, "workspace too small: %zu < %zu bytes", ws_bytes, pl.ws_bytes);
    SSQ_REQUIRE(pl.ws_bytes == 0 || workspace, "workspace is NULL");
    ContigParams cp;
    cp.a = *a;
    if (a->code_bits == 8) {  // 8-bit words are the byte rows: byte strides, the byte-code path
        cp.a.c_sb *= 4; cp.a.c_sh *= 4; cp.a.c_st *= 4;
        cp.a.code_bits = 0;
    }
    cp.G = a->num_q_heads / a->num_kv_heads;
    cp.rows = cp.G * a->q_len;
    cp.split_len = pl.split_len;
    cp.n_splits = pl.n_splits;
    const size_t n_rows_all = (size_t)a->batch * a->num_q_heads * a->q_len;
    float* ws = reinterpret_cast<float*>(workspace);
    cp.ws_o = ws;
    cp.ws_m = ws ? ws + (size_t)pl.n_splits * n_rows_all * a->value_dim : nullptr;
    cp.ws_l = ws ? cp.ws_m + (size_t)pl.n_splits * n_rows_all : nullptr;
    // passthrough dims: heavy blocks ascending, then d; record slot = block (dense) or ordinal
    const PtLayout L = pt_layout(*a);
    cp.n_hd = L.n_hd;
    cp.pt_vec = L.vec;
    for (int i = 0; i < kHP; ++i) { cp.hoff[i] = L.hoff[i]; cp.hdim[i] = L.hdim[i]; }
    int rc;
    if (!has_v) {
        rc = launch_hv<4, SSQ_BF16, false>(cp, pl, st);
    } else if (a->v_dtype == SSQ_BF16) {
        rc = pl.DT == 4 ? launch_hv<4, SSQ_BF16, true>(cp, pl, st) : launch_hv<8, SSQ_BF16, true>(cp, pl, st);
    } else {
        rc = pl.DT == 4 ? launch_hv<4, SSQ_F16, true>(cp, pl, st) : launch_hv<8, SSQ_F16, true>(cp, pl, st);
    }
    if (rc) return rc;
    if (has_v && pl.n_splits > 1) return ssq_launch_merge(*a, pl.n_splits, cp.ws_o, cp.ws_m, cp.ws_l, st);
    return SSQ_OK;
}
