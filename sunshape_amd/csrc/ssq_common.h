// Shared device/host helpers for the sunshape_amd HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sunshape_amd.h"

#define SSQ_WAVE 64

// Online softmax of the decode kernels: a row's running maximum may lag the scores seen by up to
// this much (nats) before it is raised, so most tiles skip the cross-lane maxima and the
// accumulator rescale; probabilities exp(s - m) then stay below e^8.
constexpr float kSoftmaxSlack = 8.f;

// ---------------------------------------------------------------------------
// scalar conversions (bf16 / f16 stored as raw 16-bit words)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float ssq_bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// round-to-nearest-even, as torch's float -> bfloat16 conversion (finite inputs)
__device__ __forceinline__ uint32_t ssq_f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float ssq_f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ uint32_t ssq_f32_to_f16(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// load element i of a tensor of dtype `dt` as fp32
__device__ __forceinline__ float ssq_load_elem(const void* p, int dt, int64_t i) {
    if (dt == SSQ_F32) return reinterpret_cast<const float*>(p)[i];
    uint32_t h = reinterpret_cast<const uint16_t*>(p)[i];
    return dt == SSQ_BF16 ? ssq_bf16_to_f32(h) : ssq_f16_to_f32(h);
}

// Load N elements of a tensor of dtype `dt` as fp32.  One uniform branch on the dtype surrounds
// the whole batch, so all N loads are in flight together (a branch per element makes the compiler
// wait for each load before the next one).  Every idx[i] must be a valid element offset.
template <int N>
__device__ __forceinline__ void ssq_load_elems(const void* p, int dt, const int64_t (&idx)[N], float (&out)[N]) {
    if (dt == SSQ_F32) {
        const float* f = reinterpret_cast<const float*>(p);
#pragma unroll
        for (int i = 0; i < N; ++i) out[i] = f[idx[i]];
    } else {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
        uint32_t r[N];
#pragma unroll
        for (int i = 0; i < N; ++i) r[i] = h[idx[i]];
        if (dt == SSQ_BF16) {
#pragma unroll
            for (int i = 0; i < N; ++i) out[i] = ssq_bf16_to_f32(r[i]);
        } else {
#pragma unroll
            for (int i = 0; i < N; ++i) out[i] = ssq_f16_to_f32(r[i]);
        }
    }
}

// raw bits of element i (fp32 bits, or the 16-bit pattern zero-extended); ssq_bits_to_f32 converts
__device__ __forceinline__ uint32_t ssq_load_bits(const void* p, int dt, int64_t i) {
    return dt == SSQ_F32 ? reinterpret_cast<const uint32_t*>(p)[i] : (uint32_t)reinterpret_cast<const uint16_t*>(p)[i];
}
__device__ __forceinline__ float ssq_bits_to_f32(uint32_t u, int dt) {
    return dt == SSQ_F32 ? __uint_as_float(u) : dt == SSQ_BF16 ? ssq_bf16_to_f32(u) : ssq_f16_to_f32(u);
}

// round an fp32 value to dtype `dt` and return it as fp32 (query scaling semantics)
__device__ __forceinline__ float ssq_round_to(float x, int dt) {
    if (dt == SSQ_BF16) return ssq_bf16_to_f32(ssq_f32_to_bf16(x));
    if (dt == SSQ_F16) return ssq_f16_to_f32(ssq_f32_to_f16(x));
    return x;
}

__device__ __forceinline__ void ssq_store_elem(void* p, int dt, int64_t i, float x) {
    if (dt == SSQ_F32) {
        reinterpret_cast<float*>(p)[i] = x;
    } else {
        uint32_t h = dt == SSQ_BF16 ? ssq_f32_to_bf16(x) : ssq_f32_to_f16(x);
        reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)h;
    }
}

// The keys of an encode launch.  Short sequences are folded: all sequences of one KV head share
// one key index range, i = b * seq_len + s, and gridDim.y counts KV heads, so a decode step's
// one key per sequence fills workgroups instead of giving each its own.  Otherwise gridDim.y
// counts (batch, KV head) pairs and i = s.
struct SsqKeyMap {
    int fold, b_blk, kv, n_keys;
    __device__ __forceinline__ SsqKeyMap(const ssq_encode_args& a, int fold_) : fold(fold_) {
        const int y = blockIdx.y;
        kv = fold ? y : y % a.num_kv_heads;
        b_blk = fold ? 0 : y / a.num_kv_heads;
        n_keys = fold ? a.batch * a.seq_len : a.seq_len;
    }
    // a kernel that orders its workgroups itself names the KV head and the sequence (ignored
    // when folded)
    __device__ __forceinline__ SsqKeyMap(const ssq_encode_args& a, int fold_, int kv_, int b_)
        : fold(fold_), b_blk(fold_ ? 0 : b_), kv(kv_), n_keys(fold_ ? a.batch * a.seq_len : a.seq_len) {}
    __device__ __forceinline__ void bs(const ssq_encode_args& a, int i, int& b, int& s) const {
        if (fold) {
            b = i / a.seq_len;
            s = i - b * a.seq_len;
        } else {
            b = b_blk;
            s = i;
        }
    }
    // element offset of key i's row
    __device__ __forceinline__ int64_t krow(const ssq_encode_args& a, int i) const {
        int b, s;
        bs(a, i, b, s);
        return (int64_t)b * a.k_sb + (int64_t)kv * a.k_sh + (int64_t)s * a.k_ss;
    }
};
// folding applies when a sequence is shorter than one workgroup's keys
inline bool ssq_encode_fold(const ssq_encode_args* a, int keys_per_wg) {
    return a->seq_len < keys_per_wg && (int64_t)a->batch * a->seq_len <= 0x7fffffff;
}

// Stored code width in bytes, as the reference's _compact_index_dtype (sunshape/codec.py:78-83):
// one byte up to 256 codewords, 16 bits up to 65535, 32 bits beyond.  16-bit codes are read as
// unsigned, so every index below 65536 round-trips (the reference's int16 storage holds indices up
// to 32767 as the same bits).
constexpr int kMaxCentroids = SSQ_MAX_CENTROIDS;
__host__ __device__ inline int ssq_code_width(int n_centroids) {
    return n_centroids <= 256 ? 1 : n_centroids <= 65535 ? 2 : 4;
}
// code element i (in units of the code width) of a row buffer
__device__ __forceinline__ uint32_t ssq_load_code(const uint8_t* codes, int width, int64_t i) {
    return width == 1 ? (uint32_t)codes[i]
                      : width == 2 ? (uint32_t)reinterpret_cast<const uint16_t*>(codes)[i]
                                   : reinterpret_cast<const uint32_t*>(codes)[i];
}

__device__ __forceinline__ bool ssq_is_heavy(const uint64_t hm0, const uint64_t hm1, int blk) {
    return blk < 64 ? ((hm0 >> blk) & 1ull) : ((hm1 >> (blk - 64)) & 1ull);
}

// wave64 reductions through ds_swizzle/bpermute (__shfl_xor)
__device__ __forceinline__ float ssq_wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, SSQ_WAVE));
    return v;
}
__device__ __forceinline__ float ssq_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, SSQ_WAVE);
    return v;
}

// ---------------------------------------------------------------------------
// host-side error plumbing
// ---------------------------------------------------------------------------
int ssq_fail(int code, const char* fmt, ...);
int ssq_check_hip(hipError_t e, const char* what);
// allow `bytes` of dynamic LDS for kernel `fn` on the current device (set once per kernel and device)
int ssq_allow_lds(const void* fn, int bytes, const char* what);

// compute units of the current device (cached per device; 256 on MI355X)
int ssq_device_cus();
// grid-search encode (ssq_encode_grid.hip)
bool ssq_encode_grid_supported(const ssq_encode_args* a);
int ssq_encode_grid_run(const ssq_encode_args* a, hipStream_t st);
// exact encode for codebooks of more than 256 codewords (ssq_encode_wide.hip)
int ssq_encode_wide_run(const ssq_encode_args* a, hipStream_t st);

#define SSQ_REQUIRE(cond, ...)                                  \
    do {                                                        \
        if (!(cond)) return ssq_fail(SSQ_ERR_INVALID, __VA_ARGS__); \
    } while (0)
#define SSQ_UNSUPPORTED(cond, ...)                                  \
    do {                                                            \
        if (!(cond)) return ssq_fail(SSQ_ERR_UNSUPPORTED, __VA_ARGS__); \
    } while (0)
