// Pieces shared by the paged decode kernels (ssq_decode_mfma.h: LUT scores;
// ssq_decode_paged_q4.hip: 4x4 MFMA scores): launch shape, parameters, the wave reductions, and the
// 64-token tile loads (one token's codes per lane, V fragments straight from the dim-major pages).
#pragma once

#include "ssq_common.h"

// Parameters of one paged decode launch (shared type: both kernels' host code fills it)
struct SsqPagedParams {
    ssq_decode_args a;
    int G, rows, split_len, n_splits;
    int rg;  // query rows per row group (blockIdx.z)
    // passthrough dims of the contiguous LUT kernel: n_hd (<= 16) dims, each at element hoff[i] of
    // a token's passthrough row and permuted query dim hdim[i]
    int n_hd;
    int hoff[16], hdim[16];
    int pt_vec;  // the n_hd (8 or 16) values are consecutive 16-bit elements, 16-byte aligned (the
                 // contiguous LUT kernel's passthrough variant requires it)
    float* ws_o;
    float* ws_m;
    float* ws_l;
};

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

#ifndef SSQ_DECODE_WAVES
#define SSQ_DECODE_WAVES 4
#endif
constexpr int kWaves = SSQ_DECODE_WAVES;  // waves per workgroup
constexpr int kThreads = kWaves * SSQ_WAVE;
constexpr int kTileTok = 64;  // tokens per wave iteration (4 pages)
constexpr int kPage = 16;
constexpr int kNC = 256;      // codewords per block (uint8 codes)
constexpr size_t kMaxSmem = 160 * 1024;

using MfmaParams = SsqPagedParams;


typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// round to the value dtype (round to nearest even; gfx950's v_cvt_pk_bf16_f32 for bf16)
template <int VT>
__device__ __forceinline__ uint32_t to_vt16(float x) {
    if constexpr (VT == SSQ_BF16) {
        const bf16x2_t r = __builtin_convertvector((f32x2_t){x, 0.f}, bf16x2_t);
        return __builtin_bit_cast(uint32_t, r) & 0xFFFFu;
    } else {
        return ssq_f32_to_f16(x);
    }
}

template <int VT>
__device__ __forceinline__ v4f mfma(const uint4& a, const uint4& b, v4f c) {
    if (VT == SSQ_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0,
                                                       0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
}

// wave-wide max / sum: DPP rotations inside each 16-lane row, then the four row results by readlane
template <int CTL>
__device__ __forceinline__ float dpp_ror(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_ror<0x121>(v));
    v = fmaxf(v, dpp_ror<0x122>(v));
    v = fmaxf(v, dpp_ror<0x124>(v));
    v = fmaxf(v, dpp_ror<0x128>(v));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_ror<0x121>(v);
    v += dpp_ror<0x122>(v);
    v += dpp_ror<0x124>(v);
    v += dpp_ror<0x128>(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// 16-byte load of streamed (read-once) data: non-temporal, so the single pass over
// the values does not evict the codebooks and block tables other workgroups reuse
#ifndef SSQ_STREAM_NT
#define SSQ_STREAM_NT 1
#endif
#ifndef SSQ_CODES_NT
#define SSQ_CODES_NT 1
#endif
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const uint16_t* p) {
#if SSQ_STREAM_NT
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
#else
    return *reinterpret_cast<const uint4*>(p);
#endif
}

// packed code rows (PB bits per code, 32 / PB codes per little-endian int32 word, the low bits
// first; sunshape/triton_kernels.py:250-266): int32 words per row
__host__ __device__ constexpr int pk_words(int NB, int PB) { return PB ? (NB + 32 / PB - 1) / (32 / PB) : 1; }

// registers of one 64-token tile in flight
template <int NB, int DT, int PB = 0>
struct TileRegs {
    uint4 c[NB / 16 > 0 ? NB / 16 : 1];  // this lane's token codes (NB bytes)
    uint2 c8;                            // NB == 8
    uint32_t pk[pk_words(NB, PB)];       // PB-bit codes in words (PB > 0)
    uint4 v[2][DT];                      // B-operand V fragments of the two 32-token K groups
};

// cbase: the KV head's codes (bytes; with PB > 0 int32 words, strides counting words)
template <int NB, int DT, int PB = 0>
__device__ __forceinline__ void issue_tile(const ssq_decode_args& a, const int* pages, int t_begin, int t_end, int tile,
                                           int lane, const uint8_t* cbase, const uint16_t* vbase,
                                           TileRegs<NB, DT, PB>& R) {
    // Every load is issued unconditionally (straight-line code keeps the compiler's vmcnt
    // bookkeeping exact, so waiting for this tile never drains the next one).  Lanes past the
    // split's end read their split's last token / 8-token chunk instead: a valid address whose
    // data compute_tile masks (scores by `valid`, V chunks by the tail zeroing).
    const int rel = tile * kTileTok;  // tile start relative to the split
    const int last = t_end - 1 - t_begin;
    const int tr = min(rel + lane, last);
    const int page = pages[tr >> 4];
    const uint8_t* crow = cbase + (int64_t)page * a.c_sb + (int64_t)((t_begin + tr) & 15) * a.c_st;
    if constexpr (PB > 0) {
        const uint32_t* prow = reinterpret_cast<const uint32_t*>(cbase) + (int64_t)page * a.c_sb +
                               (int64_t)((t_begin + tr) & 15) * a.c_st;
#pragma unroll
        for (int i = 0; i < pk_words(NB, PB); ++i) R.pk[i] = __builtin_nontemporal_load(prow + i);
    } else if (NB >= 16) {
#pragma unroll
        for (int i = 0; i < NB / 16; ++i) {
#if SSQ_CODES_NT
            const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(crow) + i);
            R.c[i] = make_uint4(v.x, v.y, v.z, v.w);
#else
            R.c[i] = reinterpret_cast<const uint4*>(crow)[i];
#endif
        }
    } else {
        R.c8 = *reinterpret_cast<const uint2*>(crow);
    }
    const int kchunk = 8 * (lane >> 4);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        const int r = min(rel + 32 * g + kchunk, last & ~7);
        const uint16_t* src = vbase + (int64_t)pages[r >> 4] * a.v_sb + (r & 15);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) R.v[g][dt] = load_stream(src + (int64_t)(16 * dt) * a.v_st);
    }
}

// the raw-score store of a tile's scores s[r] (row r, this lane's token t0 + lane), if requested
template <int RP>
__device__ __forceinline__ void tile_store_scores(const MfmaParams& p, int b, int kv, int t0, int t_end, int lane,
                                                  const float (&s)[RP]) {
    const ssq_decode_args& a = p.a;
    const int t = t0 + lane;
    if (t < t_end) {
        if (a.scores) {
            const int row0 = blockIdx.z * p.rg, nr = min(p.rg, p.rows - row0);
#pragma unroll
            for (int r = 0; r < RP; ++r) {
                if (r < nr) {
                    const int g = (row0 + r) / a.q_len, qi = row0 + r - g * a.q_len;
                    const int h = kv * p.G + g;
                    a.scores[(int64_t)b * a.s_sb + (int64_t)h * a.s_sh + (int64_t)qi * a.s_sl + t] = s[r];
                }
            }
        }
    }
}

// After a tile's scores s[r] (row r, this lane's token t0 + lane): the raw-score store, the online
// softmax update (wave-local) and the probabilities cast to the value dtype in the wave's P strip
// [RP][64], visible to the whole wave on return.
template <int RP, int DT, int VT>
__device__ __forceinline__ void tile_probs(const MfmaParams& p, uint16_t* pstrip, int b, int kv, int t0, int t_end,
                                           int lane, const float (&s)[RP], float (&m_run)[RP], float (&l_lane)[RP],
                                           v4f (&acc)[DT]) {
    tile_store_scores<RP>(p, b, kv, t0, t_end, lane, s);
    const bool valid = t0 + lane < t_end;
    // online softmax (wave-local).  The running maximum m_run[r] is wave-uniform and moves only
    // when some score of the tile exceeds it by more than kSoftmaxSlack: most tiles skip the
    // cross-lane maxima and the accumulator rescale.
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
            const float mn = fmaxf(m_run[r], wave_max(sv[r]));
            alpha[r] = mn == -INFINITY ? 1.f : __expf(m_run[r] - mn);
            l_lane[r] *= alpha[r];
            m_run[r] = mn;
        }
        // accumulator row 4 g + i lives in lane group g = lane / 16
        const int grp = lane >> 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float f = 1.f;
#pragma unroll
            for (int g = 0; g < 4; ++g)
                if (4 * g + i < RP) f = grp == g ? alpha[4 * g + i] : f;
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
        pstrip[r * kTileTok + lane] = (uint16_t)to_vt16<VT>(pr);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// tile_probs, then P.V on v_mfma_f32_16x16x32 with V fragments from the tile's registers
template <int RP, int DT, int VT, int NB, int PB>
__device__ __forceinline__ void tile_softmax_pv(const MfmaParams& p, uint16_t* pstrip, int b, int kv, int t0, int t_end,
                                                int lane, const float (&s)[RP], TileRegs<NB, DT, PB>& R,
                                                float (&m_run)[RP], float (&l_lane)[RP], v4f (&acc)[DT]) {
    tile_probs<RP, DT, VT>(p, pstrip, b, kv, t0, t_end, lane, s, m_run, l_lane, acc);
    const int arow = lane & 15;
    const int kchunk = 8 * (lane >> 4);
    const bool tail = t0 + kTileTok > t_end;  // wave-uniform: the tile holds the split's end
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        const int tk = t0 + 32 * g + kchunk;
        uint4 af = make_uint4(0, 0, 0, 0);
        if (arow < RP) af = *reinterpret_cast<const uint4*>(pstrip + arow * kTileTok + 32 * g + kchunk);
        if (tail && tk + 8 > t_end) {  // values of slots past the end are unwritten; zero them
            const int keep = t_end - tk;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                uint32_t w[4] = {R.v[g][dt].x, R.v[g][dt].y, R.v[g][dt].z, R.v[g][dt].w};
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (j >= keep) w[j >> 1] &= (j & 1) ? 0x0000FFFFu : 0xFFFF0000u;
                R.v[g][dt] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] = mfma<VT>(af, R.v[g][dt], acc[dt]);
    }
    __builtin_amdgcn_wave_barrier();
}

}  // namespace
