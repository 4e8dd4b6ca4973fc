// VQ-key decode for 16-bit codes (4,096 codewords of dim 4 at 3 bits/dim, 1,024 of dim 2 at 5, ...)
// over long contexts: the codebook staged in LDS one block at a time for a super-tile of tokens.
//
// The per-token path (k_decode_generic, 16-bit-code variants) gathers each token's codeword of each
// block from the codebook in memory: one random 16-byte read per (token, block), an L2 line each,
// and the gathers bound it.  Here a workgroup takes a super-tile of 4,096 tokens of one
// (batch, KV head) and walks the blocks in order: block blk's codebook (nc * bd floats, at most
// 64 KiB) is copied into LDS once, every token's codeword of that block is read from there, and
// its scores (one per query row, at most 4 rows per workgroup) are accumulated in registers.
// Block blk + 1's codebook goes into the other half of a double buffer while blk is computed
// (direct global-to-LDS loads issued before blk's arithmetic), so one workgroup barrier per
// block separates them.  The score arithmetic is the per-token path's (the LUT entry's FMA chain
// over the block's dims from the first product, blocks added in order), so the raw scores equal it
// bit for bit.
//
// Then per super-tile: mask, optional raw-score store, the softmax update (the super-tile's row
// maximum), P.V over the super-tile's V rows (streamed, 16 loads in flight per thread), and at the
// end of the split the normalised output + lse, or (m, l, o) partials for k_merge -- the same
// outputs and workspace layout as k_decode_generic (sunshape/vllm_attn_backend.py:216-253; scores
// sunshape/triton_kernels.py:174-196, LUT entries :381-408).
//
// 512 threads (8 waves), one workgroup per CU (the double buffer is 128 KiB at 4,096 codewords of
// dim 4).  Host-checked: 16-bit codes in 16-byte aligned rows of a multiple of 8 blocks (at most
// 64), codewords of 2 or 4 dims in a 16-byte aligned codebook of at most 64 KiB per block, no
// passthrough blocks, bf16 or f16 values of 64 or 128 dims.
#include "ssq_decode_generic.h"

namespace {

constexpr int kWT = 512;                 // threads per workgroup
constexpr int kWWaves = kWT / SSQ_WAVE;  // 8
constexpr int kPD = 4;                   // value dims per thread in the paged P.V

// tokens per thread per super-tile (the super-tile is kWT times that); at most 4 query rows per
// workgroup (more rows take further workgroups)
__host__ __device__ constexpr int wide_tpt(int) { return 8; }

// LDS layout, in floats: [stage / p / obuf | qp | red | pgl]
struct WideLds {
    size_t qp, red, pgl, total;
};
__host__ __device__ inline WideLds wide_lds(const ssq_decode_args& a, int RP) {
    const size_t ncb = (size_t)a.n_centroids * a.block_dim;
    const size_t sup = (size_t)wide_tpt(RP) * kWT;
    size_t r0 = 2 * ncb;                                              // double-buffered codebook stage
    if ((size_t)RP * sup > r0) r0 = (size_t)RP * sup;                 // the super-tile's p
    if ((size_t)kWWaves * RP * a.value_dim > r0) r0 = (size_t)kWWaves * RP * a.value_dim;  // epilogue
    if ((size_t)kWT * kPD * RP > r0) r0 = (size_t)kWT * kPD * RP;     // paged epilogue: kWT*kPD/Dv slots
    WideLds l;
    l.qp = (r0 + 3) & ~(size_t)3;
    l.red = l.qp + (size_t)RP * a.head_dim;
    l.pgl = l.red + 2 * kWWaves * RP;
    l.total = l.pgl + sup / 8;
    return l;
}

// One block's codebook (n4 16-byte pieces, at most 8 * kWT) into an LDS stage half with direct
// global-to-LDS loads: wave w's u-th load puts its 64 lanes' pieces u * kWT + 64 w + lane at the
// wave's LDS base + 16 * lane (lanes past n4 are inactive).  Completion is waited for with vmcnt.
__device__ __forceinline__ void stage_block_lds(const float* src_blk, float* half, int n4, int tid) {
    const int wbase = tid & ~(SSQ_WAVE - 1);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int i = u * kWT + tid;
        if (i < n4)
            __builtin_amdgcn_global_load_lds(static_cast<const void*>(src_blk + (size_t)i * 4),
                                             (__attribute__((address_space(3))) void*)(half + (size_t)(u * kWT + wbase) * 4),
                                             16, 0, 0);
    }
}

// BD: the block dim, 2 or 4 (the plan's condition), fixed at compile time so that each token's
// codeword is one LDS read and its FMA chain carries no branches
template <int RP, bool PAGED, int VT, int BD>
__global__ __launch_bounds__(kWT) void k_decode_wide(const SsqGenericParams p) {
    extern __shared__ __align__(16) float smem[];
    const ssq_decode_args& a = p.a;
    constexpr int kK = wide_tpt(RP);
    constexpr int kSup = kK * kWT;
    const WideLds L = wide_lds(a, RP);
    const int tid = threadIdx.x;
    const int lane = tid & (SSQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / SSQ_WAVE);
    const int split = blockIdx.x;
    const int grp = blockIdx.y;
    const int bk = blockIdx.z;
    const int b = bk / a.num_kv_heads;
    const int kv = bk - b * a.num_kv_heads;
    const int nb = a.n_blocks, nc = a.n_centroids, D = a.head_dim, Dv = a.value_dim;
    constexpr int bd = BD;
    const int r0 = grp * p.R;
    const int nr = min(p.R, p.rows - r0);
    const int T = PAGED ? min(a.seq_lens[b], a.seq_len) : a.seq_len;
    const int t_begin = split * p.split_len;
    const int t_end = min(T, t_begin + p.split_len);
    const int ncb = nc * bd;
    const int n4 = ncb / 4;  // float4s of one block's codebook: at most 8 per thread (host-checked)
    float* stage = smem;     // [2][ncb]
    float* pbuf = smem;      // [RP][kSup], after a super-tile's blocks
    float* qp = smem + L.qp;
    float* red = smem + L.red;
    int* pgl = reinterpret_cast<int*>(smem + L.pgl);

    // ---- scaled, permuted query rows (as k_decode_generic)
    const int64_t* perm = a.perm + (int64_t)kv * a.perm_sh;
    for (int e0 = 0; e0 < RP * D; e0 += 4 * kWT) {
        int64_t src[4];
        bool ok[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = e0 + k * kWT + tid;
            src[k] = perm[e < RP * D ? e % D : 0];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = e0 + k * kWT + tid;
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
            const int e = e0 + k * kWT + tid;
            if (e < RP * D) qp[e] = !ok[k] ? 0.f : a.has_scale ? ssq_round_to(v[k] * a.scale, a.q_dtype) : v[k];
        }
    }

    const float* cent = a.cent + (int64_t)kv * a.cent_sh;
    const uint16_t* codes = reinterpret_cast<const uint16_t*>(a.codes);
    float m_run[RP], l_thr[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) { m_run[r] = -INFINITY; l_thr[r] = 0.f; }
    // P.V mapping: contiguous rows, 8 dims of one token per thread and load; pages [P, Hkv, Dv,
    // page], 8 tokens of one dim per load and kPD dims per thread, pv_d + dd * dchunks (one read of
    // the chunk's p for kPD loads; a load's lanes stay on consecutive dims)
    constexpr int kAccW = PAGED ? kPD : 8;
    const int dchunks = PAGED ? Dv / kPD : Dv / 8;
    const int tpar = kWT / dchunks;
    const int pv_t = tid / dchunks;
    const int pv_d = tid - pv_t * dchunks;
    float acc[RP][kAccW];
#pragma unroll
    for (int r = 0; r < RP; ++r)
#pragma unroll
        for (int j = 0; j < kAccW; ++j) acc[r][j] = 0.f;

    for (int T0 = t_begin; T0 < t_end; T0 += kSup) {
        // this thread's tokens T0 + k * kWT + tid (past t_end: the last token's row, not used);
        // pages: the page of each 8-token chunk into pgl (page_size % 8 == 0), for the code rows
        // and the P.V loads
        if (PAGED) {
            for (int c = tid; c < kSup / 8; c += kWT) {
                const int t = min(T0 + 8 * c, t_end - 1);
                pgl[c] = a.block_table[(int64_t)b * a.bt_sb + t / a.page_size];
            }
            __syncthreads();  // the page list is read below (code rows) by other threads
        }
        // the code row (16-bit elements) of this thread's k-th token
        auto code_row = [&](int k) -> int64_t {
            const int tt = k * kWT + tid;
            const int t = min(T0 + tt, t_end - 1);
            if (PAGED) {
                const int off = t - (t / a.page_size) * a.page_size;
                return (int64_t)pgl[(t - T0) >> 3] * a.c_sb + (int64_t)kv * a.c_sh + (int64_t)off * a.c_st;
            }
            return (int64_t)b * a.c_sb + (int64_t)kv * a.c_sh + (int64_t)t * a.c_st;
        };
        float ss[kK][RP];
#pragma unroll
        for (int k = 0; k < kK; ++k)
#pragma unroll
            for (int r = 0; r < RP; ++r) ss[k][r] = 0.f;

        // 8 blocks' codes of each token: one 16-byte piece of its row, the first one loaded beside
        // block 0's codebook copy into stage half 0 (the previous super-tile's p reads are done: the
        // barrier that ended its P.V)
        ssq_v4u w[kK];
#pragma unroll
        for (int k = 0; k < kK; ++k) w[k] = *reinterpret_cast<const ssq_v4u*>(codes + code_row(k));
        stage_block_lds(cent, stage, n4, tid);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
#pragma unroll 1
        for (int blk = 0; blk < nb; ++blk) {
            const int kb = blk & 7;
            uint32_t cw[kK];  // this block's codeword of each token (w[k].x: this block pair's word)
#pragma unroll
            for (int k = 0; k < kK; ++k) {
                const uint32_t code = (kb & 1) ? (w[k].x >> 16) : (w[k].x & 0xFFFFu);
                cw[k] = code < (uint32_t)nc ? code : (uint32_t)(nc - 1);
            }
            if (kb == 7) {  // w is spent: the next 8 blocks' piece loads during this block's arithmetic
                if (blk + 1 < nb) {
#pragma unroll
                    for (int k = 0; k < kK; ++k) w[k] = *reinterpret_cast<const ssq_v4u*>(codes + code_row(k) + blk + 1);
                }
            } else if (kb & 1) {  // the next pair's codes move to .x
#pragma unroll
                for (int k = 0; k < kK; ++k) w[k] = ssq_v4u{w[k].y, w[k].z, w[k].w, 0u};
            }
            const float* cur = stage + (size_t)(blk & 1) * ncb;
            const bool more = blk + 1 < nb;
            // the next block's codebook into the other half (last read in the previous block, before
            // its barrier), in flight during this block's arithmetic
            if (more) stage_block_lds(cent + (int64_t)(blk + 1) * ncb, stage + (size_t)((blk + 1) & 1) * ncb, n4, tid);
            float qv[RP][BD];
#pragma unroll
            for (int r = 0; r < RP; ++r)
#pragma unroll
                for (int d = 0; d < BD; ++d) qv[r][d] = qp[r * D + blk * BD + d];
#pragma unroll
            for (int k = 0; k < kK; ++k) {
                const uint32_t cc = cw[k];
                float c[BD];
                if constexpr (BD == 4) {
                    const float4 v4 = *reinterpret_cast<const float4*>(cur + (size_t)cc * 4);
                    c[0] = v4.x; c[1] = v4.y; c[2] = v4.z; c[3] = v4.w;
                } else {
                    const float2 v2 = *reinterpret_cast<const float2*>(cur + (size_t)cc * 2);
                    c[0] = v2.x; c[1] = v2.y;
                }
                float e_acc[RP];
#pragma unroll
                for (int r = 0; r < RP; ++r) e_acc[r] = qv[r][0] * c[0];
#pragma unroll
                for (int d = 1; d < BD; ++d)
#pragma unroll
                    for (int r = 0; r < RP; ++r) e_acc[r] = fmaf(qv[r][d], c[d], e_acc[r]);
#pragma unroll
                for (int r = 0; r < RP; ++r) ss[k][r] += e_acc[r];
            }
            __builtin_amdgcn_s_waitcnt(0);  // the next half (and at kb 7 the next code piece) has landed
            __syncthreads();
        }

        // ---- mask, raw scores, softmax update
        float mx[RP];
#pragma unroll
        for (int r = 0; r < RP; ++r) mx[r] = -INFINITY;
#pragma unroll
        for (int k = 0; k < kK; ++k) {
            const int t = T0 + k * kWT + tid;
            const bool valid = t < t_end;
            if (valid && a.mask) {
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
                    if (r < nr) ss[k][r] += mk[r];
            }
            if (valid && a.scores) {
#pragma unroll
                for (int r = 0; r < RP; ++r) {
                    if (r < nr) {
                        const int row = r0 + r;
                        const int g = row / a.q_len, qi = row - g * a.q_len;
                        const int h = kv * p.G + g;
                        a.scores[(int64_t)b * a.s_sb + (int64_t)h * a.s_sh + (int64_t)qi * a.s_sl + t] = ss[k][r];
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < RP; ++r) mx[r] = fmaxf(mx[r], valid ? ss[k][r] : -INFINITY);
        }
#pragma unroll
        for (int r = 0; r < RP; ++r) {
            const float v = ssq_wave_max(mx[r]);
            if (lane == 0) red[wave * RP + r] = v;
        }
        __syncthreads();
        float alpha[RP];
#pragma unroll
        for (int r = 0; r < RP; ++r) {
            float tm = red[r];
#pragma unroll
            for (int w2 = 1; w2 < kWWaves; ++w2) tm = fmaxf(tm, red[w2 * RP + r]);
            const float mn = fmaxf(m_run[r], tm);
            alpha[r] = (mn == -INFINITY) ? 1.f : __expf(m_run[r] - mn);
            m_run[r] = mn;
            float lsum = 0.f;
#pragma unroll
            for (int k = 0; k < kK; ++k) {
                const int tt = k * kWT + tid;
                const float pr = (T0 + tt < t_end && mn != -INFINITY) ? __expf(ss[k][r] - mn) : 0.f;
                lsum += pr;
                pbuf[(size_t)r * kSup + tt] = pr;
            }
            l_thr[r] = l_thr[r] * alpha[r] + lsum;
        }
#pragma unroll
        for (int r = 0; r < RP; ++r)
#pragma unroll
            for (int j = 0; j < kAccW; ++j) acc[r][j] *= alpha[r];
        __syncthreads();

        // ---- P.V over the super-tile's nt tokens: 16 loads per thread issued before their
        // arithmetic (indexes clamped to the last token / chunk; the clamped slots are skipped)
        const int nt = min(kSup, t_end - T0);
        constexpr int kVB = 16;
        if (!PAGED) {
            const int64_t vbase = (int64_t)b * a.v_sb + (int64_t)kv * a.v_sh + pv_d * 8;
            for (int tt0 = pv_t; tt0 < nt; tt0 += kVB * tpar) {
                VRaw8<VT> raw[kVB];
#pragma unroll
                for (int k = 0; k < kVB; ++k)
                    raw[k] = load_v8_raw<VT, true>(a.v, vbase + (int64_t)(T0 + min(tt0 + k * tpar, nt - 1)) * a.v_st);
                __asm__ volatile("" ::: "memory");  // the batch's loads stay ahead of every use
#pragma unroll
                for (int k = 0; k < kVB; ++k) {
                    const int tt = tt0 + k * tpar;
                    if (tt >= nt) break;
                    float v[8];
                    unpack_v8<VT>(raw[k], v);
#pragma unroll
                    for (int r = 0; r < RP; ++r) {
                        const float pr = pbuf[(size_t)r * kSup + tt];
#pragma unroll
                        for (int j = 0; j < 8; ++j) acc[r][j] = fmaf(pr, v[j], acc[r][j]);
                    }
                }
            }
        } else {
            // 8-token chunks in pairs: a thread loads both halves of a 16-token run of its dim back
            // to back, so the run's line is fetched once
            const int nchunks = (nt + 7) >> 3;
            const int npairs = (nchunks + 1) >> 1;
            // load k of a batch: pair q = k / (2 kPD), dim dd = (k / 2) % kPD, half h = k % 2
            constexpr int kPairs = kVB / (2 * kPD);
            const int64_t vhead = (int64_t)kv * a.v_sh + (int64_t)pv_d * a.v_st;
            for (int c0 = pv_t; c0 < npairs; c0 += kPairs * tpar) {
                VRaw8<VT> raw[kVB];
#pragma unroll
                for (int k = 0; k < kVB; ++k) {
                    const int q = k / (2 * kPD), dd = (k >> 1) % kPD;
                    const int tt = min(2 * (c0 + q * tpar) + (k & 1), nchunks - 1) * 8;
                    const int t = T0 + tt;
                    const int off = t - (t / a.page_size) * a.page_size;
                    raw[k] = load_v8_raw<VT, true>(a.v, (int64_t)pgl[tt >> 3] * a.v_sb + vhead + (int64_t)(dd * dchunks) * a.v_st + off);
                }
                __asm__ volatile("" ::: "memory");  // the batch's loads stay ahead of every use
#pragma unroll
                for (int q = 0; q < kPairs; ++q) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int ch = 2 * (c0 + q * tpar) + h;  // increasing in (q, h)
                        if (ch >= nchunks) break;
                        const int tt = ch * 8;
                        float4 p0[RP], p1[RP];
#pragma unroll
                        for (int r = 0; r < RP; ++r) {
                            p0[r] = *reinterpret_cast<const float4*>(pbuf + (size_t)r * kSup + tt);
                            p1[r] = *reinterpret_cast<const float4*>(pbuf + (size_t)r * kSup + tt + 4);
                        }
#pragma unroll
                        for (int dd = 0; dd < kPD; ++dd) {
                            float v[8];
                            unpack_v8<VT>(raw[(q * kPD + dd) * 2 + h], v);
#pragma unroll
                            for (int j = 0; j < 8; ++j)
                                if (tt + j >= nt) v[j] = 0.f;  // tokens past the end: p = 0 and V unwritten
#pragma unroll
                            for (int r = 0; r < RP; ++r) {
                                float x = acc[r][dd];
                                x = fmaf(p0[r].x, v[0], x); x = fmaf(p0[r].y, v[1], x);
                                x = fmaf(p0[r].z, v[2], x); x = fmaf(p0[r].w, v[3], x);
                                x = fmaf(p1[r].x, v[4], x); x = fmaf(p1[r].y, v[5], x);
                                x = fmaf(p1[r].z, v[6], x); x = fmaf(p1[r].w, v[7], x);
                                acc[r][dd] = x;
                            }
                        }
                    }
                }
            }
        }
        __syncthreads();  // p and pgl are read before the next super-tile's stage / pages
    }

    // ---- epilogue: l summed over threads; o over token lanes (contiguous: first within the wave,
    // whose lanes hold 64 / dchunks token lanes of every dim chunk), then over waves / lanes in LDS
    float* red2 = red + kWWaves * RP;
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        const float v = ssq_wave_sum(l_thr[r]);
        if (lane == 0) red2[wave * RP + r] = v;
    }
    float* obuf = smem;  // [slots][RP][Dv]
    int slots;
    if (!PAGED) {
        for (int o = dchunks; o < SSQ_WAVE; o <<= 1)
#pragma unroll
            for (int r = 0; r < RP; ++r)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[r][j] += __shfl_xor(acc[r][j], o, SSQ_WAVE);
        slots = kWWaves;
        if (lane < dchunks) {
#pragma unroll
            for (int r = 0; r < RP; ++r)
#pragma unroll
                for (int j = 0; j < 8; ++j) obuf[((size_t)wave * RP + r) * Dv + pv_d * 8 + j] = acc[r][j];
        }
    } else {
        slots = tpar;
#pragma unroll
        for (int r = 0; r < RP; ++r)
#pragma unroll
            for (int dd = 0; dd < kAccW; ++dd) obuf[((size_t)pv_t * RP + r) * Dv + pv_d + dd * dchunks] = acc[r][dd];
    }
    __syncthreads();
    const int n_rows_all = a.batch * a.num_q_heads * a.q_len;
    for (int e = tid; e < nr * Dv; e += kWT) {
        const int r = e / Dv, dv = e - r * Dv;
        float l = 0.f;
        for (int w2 = 0; w2 < kWWaves; ++w2) l += red2[w2 * RP + r];
        float o = 0.f;
        for (int s2 = 0; s2 < slots; ++s2) o += obuf[((size_t)s2 * RP + r) * Dv + dv];
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

template <int RP, bool PAGED, int VT>
int launch_wide_t(const SsqGenericParams& dp, int n_groups, size_t smem, hipStream_t st) {
    auto kern = dp.a.block_dim == 4 ? k_decode_wide<RP, PAGED, VT, 4> : k_decode_wide<RP, PAGED, VT, 2>;
    int rc = ssq_allow_lds((const void*)kern, (int)kMaxSmem, "hipFuncSetAttribute(decode wide)");
    if (rc) return rc;
    dim3 grid(dp.n_splits, n_groups, dp.a.batch * dp.a.num_kv_heads);
    hipLaunchKernelGGL(kern, grid, dim3(kWT), smem, st, dp);
    return ssq_check_hip(hipGetLastError(), "k_decode_wide launch");
}

template <int RP>
int launch_wide_rp(const SsqGenericParams& dp, int n_groups, size_t smem, hipStream_t st) {
    const bool paged = dp.a.layout == SSQ_PAGED;
    if (dp.a.v_dtype == SSQ_BF16)
        return paged ? launch_wide_t<RP, true, SSQ_BF16>(dp, n_groups, smem, st)
                     : launch_wide_t<RP, false, SSQ_BF16>(dp, n_groups, smem, st);
    return paged ? launch_wide_t<RP, true, SSQ_F16>(dp, n_groups, smem, st)
                 : launch_wide_t<RP, false, SSQ_F16>(dp, n_groups, smem, st);
}

}  // namespace

size_t ssq_decode_wide_smem(const ssq_decode_args& a, int RP) { return wide_lds(a, RP).total * sizeof(float); }

bool ssq_decode_wide_fits(const ssq_decode_args& a) {
    const size_t ncb = (size_t)a.n_centroids * a.block_dim;
    return (a.block_dim == 2 || a.block_dim == 4) && ncb % 4 == 0 && ncb / 4 <= (size_t)8 * kWT &&
           (a.value_dim == 64 || a.value_dim == 128) &&
           (a.v_dtype == SSQ_BF16 || a.v_dtype == SSQ_F16);
}

int ssq_decode_wide(const SsqGenericParams& dp, int RP, int n_groups, size_t smem, hipStream_t st) {
    switch (RP) {
        case 1: return launch_wide_rp<1>(dp, n_groups, smem, st);
        case 2: return launch_wide_rp<2>(dp, n_groups, smem, st);
        default: return launch_wide_rp<4>(dp, n_groups, smem, st);
    }
}
