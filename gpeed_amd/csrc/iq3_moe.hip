// Routed-expert (MoE) path on the GPU (gfx950), model_batch.cpp:165-262.
//
// k_moe_route    router top-k per token, expert histogram, exclusive scan and
//                a stable scatter of the (token, k) assignments into expert
//                buckets: eptr / tok / wt exactly as the CPU builds them.
// k_moe_plan     expert buckets -> work segments of at most 8 tokens
//                (numbered heaviest first), the segment of every bucket
//                slot, each token's slots in expert order; zeroes the work
//                counters.
// k_prep_grouped gathers each slot's activation (MODE 0: X[tok], MODE 1:
//                SwiGLU of the gate/up rows) into its segment's prepared
//                activation.
// k_gemv_grouped ragged grouped GEMV: a wavefront takes (segment, tensor,
//                tile) items (its first by its index, the others from an
//                atomic counter) and streams the tile's records over the
//                whole row (no partial sums leave it).
// k_moe_combine  Y[t] = sum over the token's slots, in expert order, of
//                wt * down row (one fma per term, like axpy_f32).
#include <algorithm>
#include <climits>
#include <type_traits>

#include "iq3_common.h"
#include "iq3_gemv_core.h"
#include "iq3_kernels.h"
#include "iq3_prof.h"

namespace gpeed {

namespace {

constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 32;
constexpr int kSegTok = 8;
constexpr int kPlanMaxTok = 8192;  // tokens per routed batch (plan's per-token counters live in LDS)

// ---------------------------------------------------------------------------
// Router

// Rank order of (key, id) pairs: larger key first, equal keys lower id
// first, as one unsigned 64-bit number (larger ranks first): the
// key's bits made monotonic (non-NaN keys, -0 taken as +0), then the
// complemented id. 0 ranks after every candidate.
__device__ __forceinline__ uint64_t rank_word(float key, int id) {
    uint32_t u = __builtin_bit_cast(uint32_t, key + 0.0f);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint32_t)~id;
}

// Largest rank word over the wavefront, in every lane: DPP exchanges
// inside rows of 16 lanes, then the four row winners read back.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    auto step = [&](auto ctrl) {
        constexpr int c = decltype(ctrl)::value;
        const uint32_t hi = __builtin_amdgcn_update_dpp(0, (int)(v >> 32), c, 0xF, 0xF, false);
        const uint32_t lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, c, 0xF, 0xF, false);
        const uint64_t o = ((uint64_t)hi << 32) | lo;
        v = o > v ? o : v;
    };
    step(std::integral_constant<int, 0xB1>{});   // quad_perm [1, 0, 3, 2]
    step(std::integral_constant<int, 0x4E>{});   // quad_perm [2, 3, 0, 1]
    step(std::integral_constant<int, 0x141>{});  // row_half_mirror
    step(std::integral_constant<int, 0x140>{});  // row_mirror
    uint64_t best = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint64_t w = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), 16 * r) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 16 * r);
        best = w > best ? w : best;
    }
    return best;
}

// Exclusive scan of v[0..n) in LDS into out (n <= 1024, 1024 threads);
// returns the total. tmp: at least 17 ints of scratch. Each wavefront scans
// its 64 values with lane shuffles, the 16 wavefront totals are scanned by
// the first wavefront, and each value adds its wavefront's offset.
__device__ __forceinline__ int block_exclusive_scan(const int* v, int* out, int* tmp, int n) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int x = tid < n ? v[tid] : 0;
    int inc = x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(inc, off);
        if (lane >= off) inc += y;
    }
    if (lane == 63) tmp[wave] = inc;
    __syncthreads();
    if (wave == 0) {
        const int w = lane < 16 ? tmp[lane] : 0;
        int wi = w;
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            const int y = __shfl_up(wi, off);
            if (lane >= off) wi += y;
        }
        if (lane < 16) tmp[lane] = wi - w;  // exclusive offset of wavefront `lane`
        if (lane == 15) tmp[16] = wi;       // the total
    }
    __syncthreads();
    if (tid < n) out[tid] = tmp[wave] + inc - x;
    const int total = tmp[16];
    __syncthreads();
    return total;
}

// Assignments (token, k) kept in LDS when there are at most this many (a
// 512-token prefill chunk at top-8): the top-k loop then issues no global
// store (on gfx9 a wavefront's next global load would wait for its stores),
// and the last workgroup's bucket sort and plan run on LDS copies.
constexpr int kRouteLdsAsg = 4096;

// J = register slots per lane: expert e lives in lane e % 64, slot e / 64.
// Top-k of tokens t_first, t_first + t_step, ... (one wavefront per token):
// the ranked experts and their combine weights into out_e / out_w [T][K]
// (LDS or global), sel (optional) and, with cnt non-null, the per-expert
// counts (LDS atomics). rank_score: this wavefront's 32 floats of LDS.
template <int J>
__device__ __forceinline__ void topk_loop(const float* __restrict__ logits, int T, int E, int K, int mode,
                                          const float* __restrict__ bias, float routed_scale, int norm_topk,
                                          int* sel, int* out_e, float* out_w, int* cnt, float (*rank_score)[kMaxTopK],
                                          int t_first, int t_step, int wave, int lane) {
    // 1. top-k per token (one wavefront per token); lane l holds experts
    // l + 64j. The next token's logits are loaded while this one is ranked.
    float nxt[J];
    auto load_logits = [&](int t) {
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int e = lane + 64 * j;
            nxt[j] = (t < T && e < E) ? logits[(size_t)t * E + e] : 0.0f;
        }
    };
    load_logits(t_first);
    float bias_j[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int e = lane + 64 * j;
        bias_j[j] = (mode == 0 && bias && e < E) ? bias[e] : 0.0f;
    }
    for (int t = t_first; t < T; t += t_step) {
        float key[J], sc[J];
        uint64_t rw[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int e = lane + 64 * j;
            const float l = nxt[j];
            key[j] = -__builtin_inff();
            sc[j] = 0.0f;
            if (e < E) {
                if (mode == 0) {
                    sc[j] = 1.0f / (1.0f + expf(-l));
                    key[j] = sc[j] + bias_j[j];
                } else {
                    sc[j] = l;
                    key[j] = l;
                }
                // a NaN key ranks last (it still ranks, so every pick is an expert)
                if (__builtin_isnan(key[j])) key[j] = -__builtin_inff();
            }
            rw[j] = e < E ? rank_word(key[j], e) : 0;
        }
        load_logits(t + t_step);
        if constexpr (J == 1) {
            // rank of this lane's expert among all: one comparison per expert
            int rank = 0;
            for (int l2 = 0; l2 < E; ++l2) {  // uniform
                const uint64_t o = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(rw[0] >> 32), l2) << 32) |
                                   (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)rw[0], l2);
                rank += o > rw[0];
            }
            if (lane < E && rank < K) {
                rank_score[wave][rank] = sc[0];
                out_e[(size_t)t * K + rank] = lane;
                if (sel) sel[(size_t)t * K + rank] = lane;
                if (cnt) atomicAdd(&cnt[lane], 1);
            }
        } else {
            // K rounds: this lane's best remaining expert, then the wavefront's
            unsigned taken = 0;
            for (int k = 0; k < K; ++k) {
                uint64_t mine = 0;
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const uint64_t c = ((taken >> j) & 1u) ? 0 : rw[j];
                    mine = c > mine ? c : mine;
                }
                const int be = (int)~(uint32_t)wave_max_u64(mine);  // uniform
                float bs = 0.0f;
#pragma unroll
                for (int j = 0; j < J; ++j)
                    if ((be >> 6) == j)
                        bs = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc[j]), be & 63));
                if ((be & 63) == lane) taken |= 1u << (be >> 6);
                if (lane == 0) {
                    rank_score[wave][k] = bs;
                    out_e[(size_t)t * K + k] = be;
                    if (sel) sel[(size_t)t * K + k] = be;
                    if (cnt) atomicAdd(&cnt[be], 1);
                }
            }
        }
        // combine weights (model_batch.cpp:195-200): lane k < K takes rank
        // k; the denominator is summed in rank order. LDS writes of one
        // wavefront complete in order, so the ranks' scores are in place.
        const float s_k = lane < K ? rank_score[wave][lane] : 0.0f;
        float num = s_k;
        if (mode != 0) num = lane < K ? expf(s_k - rank_score[wave][0]) : 0.0f;
        float denom = mode == 0 ? 1e-20f : 0.0f;
        for (int k = 0; k < K; ++k)  // uniform
            denom += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, num), k));
        if (lane < K) {
            float w;
            if (mode == 0) {
                const float inv = norm_topk ? routed_scale / denom : routed_scale;
                w = s_k * inv;
            } else {
                w = num / denom;
            }
            out_w[(size_t)t * K + lane] = w;
        }
    }
}

// Exclusive scan of the expert counts into eptr and the stable scatter of
// the assignments src_e / src_w (LDS or global) into tok / wt (and the LDS
// copies l_eptr / l_tok when given). cnt, cursor, chunk_e: LDS.
__device__ __forceinline__ void bucket_body(int T, int E, int K, int* __restrict__ eptr, int* __restrict__ tok,
                                            float* __restrict__ wt, const int* src_e, const float* src_w, int* cnt,
                                            int* cursor, int* chunk_e, int* l_eptr, int* l_tok) {
    const int tid = threadIdx.x;
    // 2. exclusive scan of the expert counts (model_batch.cpp:205-209)
    {
        const int total = block_exclusive_scan(cnt, cursor, chunk_e, E);
        for (int e = tid; e < E; e += 1024) {
            eptr[e] = cursor[e];
            if (l_eptr) l_eptr[e] = cursor[e];
        }
        if (tid == 0) {
            eptr[E] = total;
            if (l_eptr) l_eptr[E] = total;
        }
    }
    __syncthreads();

    // 3. stable scatter by expert (model_batch.cpp:211-219): assignment a
    // goes to its expert's cursor plus the number of earlier assignments of
    // that expert. Per chunk of 1024 (16 wavefronts of 64, in assignment
    // order): the lanes of a wavefront with the same expert are found with
    // one ballot per bit of the expert id, a lane's rank among them is the
    // count below it; the wavefronts' counts per expert meet in a [16][64]
    // table (chunk_e), 64 experts at a time, whose column scans in wavefront
    // order give each wavefront's offset and advance the cursors.
    const int N = T * K;
    const int wave = tid >> 6, lane = tid & 63;
    const unsigned long long below = (1ull << lane) - 1ull;
    int bits = 0;
    while ((1 << bits) < E) ++bits;
    for (int c0 = 0; c0 < N; c0 += 1024) {
        const int a = c0 + tid;
        const int ea = a < N ? src_e[a] : -1;
        unsigned long long peers = __ballot(ea >= 0);
        for (int b = 0; b < bits; ++b) {
            const bool on = ea >= 0 && ((ea >> b) & 1);
            const unsigned long long m = __ballot(on);
            peers &= on ? m : ~m;
        }
        const int rank = __popcll(peers & below);
        int base = 0;
        for (int s0 = 0; s0 < E; s0 += 64) {
            chunk_e[tid] = 0;
            __syncthreads();
            const bool here = ea >= s0 && ea < s0 + 64;
            if (here && rank == 0) chunk_e[wave * 64 + (ea - s0)] = __popcll(peers);
            __syncthreads();
            if (tid < 64 && s0 + tid < E) {
                int off = cursor[s0 + tid];
                for (int w = 0; w < 16; ++w) {
                    const int c = chunk_e[w * 64 + tid];
                    chunk_e[w * 64 + tid] = off;
                    off += c;
                }
                cursor[s0 + tid] = off;
            }
            __syncthreads();
            if (here) base = chunk_e[wave * 64 + (ea - s0)];
            __syncthreads();
        }
        if (a < N) {
            const int p = base + rank;
            tok[p] = a / K;
            if (l_tok) l_tok[p] = a / K;
            wt[p] = src_w[a];
        }
    }
}


// kLds: T * K <= kRouteLdsAsg, the assignments stay in LDS.
template <int J, bool kLds>
__device__ __forceinline__ void route_body(const float* __restrict__ logits, int T, int E, int K, int mode,
                                           const float* __restrict__ bias, float routed_scale, int norm_topk,
                                           int* __restrict__ eptr, int* __restrict__ tok, float* __restrict__ wt,
                                           int* __restrict__ sel, int* __restrict__ asg_e,
                                           float* __restrict__ asg_w, int* l_eptr = nullptr,
                                           int* l_tok = nullptr) {
    __shared__ int cnt[kMaxExperts];
    __shared__ int cursor[kMaxExperts];
    __shared__ __attribute__((aligned(16))) int chunk_e[1024];
    __shared__ float rank_score[16][kMaxTopK];
    __shared__ int lds_e[kLds ? kRouteLdsAsg : 1];
    __shared__ float lds_w[kLds ? kRouteLdsAsg : 1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int e = tid; e < E; e += 1024) cnt[e] = 0;
    __syncthreads();
    int* out_e = kLds ? lds_e : asg_e;
    float* out_w = kLds ? lds_w : asg_w;
    topk_loop<J>(logits, T, E, K, mode, bias, routed_scale, norm_topk, kLds ? nullptr : sel, out_e, out_w, cnt,
                 rank_score, wave, 16, wave, lane);
    __syncthreads();
    if constexpr (kLds) {
        if (sel)
            for (int i = tid; i < T * K; i += 1024) sel[i] = lds_e[i];
    }
    bucket_body(T, E, K, eptr, tok, wt, out_e, out_w, cnt, cursor, chunk_e, l_eptr, l_tok);
}

template <int J, bool kLds>
__global__ __launch_bounds__(1024) void k_moe_route(const float* __restrict__ logits, int T, int E, int K,
                                                    int mode, const float* __restrict__ bias,
                                                    float routed_scale, int norm_topk, int* __restrict__ eptr,
                                                    int* __restrict__ tok, float* __restrict__ wt,
                                                    int* __restrict__ sel, int* __restrict__ asg_e,
                                                    float* __restrict__ asg_w) {
    route_body<J, kLds>(logits, T, E, K, mode, bias, routed_scale, norm_topk, eptr, tok, wt, sel, asg_e, asg_w);
}

// ---------------------------------------------------------------------------
// Work plan of the grouped products

struct MoePlan {
    int* n_seg;      // [1] segments, shared-expert ones first
    int* n_sh_seg;   // [1] shared-expert segments (ceil(T_sh / kSegTok))
    int* n_valid;    // [1] bucket slots to multiply: eptr[E], or 0 for buckets that break the invariants
    int* seg_e;      // [S]
    int* seg_p0;     // [S]
    int* seg_n;      // [S]
    int* seg_of;     // [N + T_sh] segment of slot p (routed bucket slots, then one per token for the shared expert)
    int* idx_of;     // [N + T_sh] token index of slot p inside its segment
    int* slot_tok;   // [N + T_sh] token of slot p (gather-mode activations)
    int* pos;        // [T][K] slots of token t, in expert order
    int* pos_tmp;    // [T][K] the same, unordered (global scratch of the stand-alone plan)
    uint32_t* ctr;   // [3] work counters (gate/up, down) and the whole-step front kernel's ticket
    uint32_t* err;   // the workspace's error word (kWsBuckets)
};

// T_sh: tokens of the shared expert (0 or T); its segments come first
// (kSegTok tokens each, all full but the last: the heaviest work), slots
// N .. N + T_sh - 1, token p - N.
// eptr / tok may be LDS copies; pos_buf (LDS, or pl.pos itself) holds the
// per-token slot lists while they are built and sorted.
// segs false (the grouped-GEMM form, which multiplies whole buckets): the
// segment tables and the slots' segment entries are not written.
__device__ __forceinline__ void plan_body(const int* eptr, const int* tok, int T, int E, int K, int T_sh, MoePlan pl,
                                          int* pos_buf, bool segs = true) {
    __shared__ int ep[kMaxExperts + 1];
    __shared__ int fstart[kMaxExperts + 1];
    __shared__ int nfull[kMaxExperts];
    __shared__ int pid[kMaxExperts];
    __shared__ int ccount[kSegTok], ccursor[kSegTok];
    __shared__ int tmp[1024];
    __shared__ int tcnt[kPlanMaxTok];
    __shared__ int bad;
    const int tid = threadIdx.x;
    for (int e = tid; e <= E; e += 1024) ep[e] = eptr[e];
    for (int t = tid; t < T; t += 1024) tcnt[t] = 0;
    if (tid < kSegTok) ccount[tid] = 0;
    if (tid == 0) bad = 0;
    __syncthreads();
    // The buckets must be what the router makes (model_batch.cpp:205-219):
    // offsets from 0, non-decreasing, ending at T*K; tokens in range, each
    // present K times. Anything else multiplies nothing: every token's
    // slots are marked empty (the combine writes zeros) and kWsBuckets is set.
    for (int e = tid; e < E; e += 1024)
        if (ep[e + 1] < ep[e]) bad = 1;
    if (tid == 0 && (ep[0] != 0 || ep[E] != T * K)) bad = 1;
    __syncthreads();
    if (!bad) {
        for (int p = tid; p < T * K; p += 1024) {
            const int t = tok[p];
            if (t < 0 || t >= T) bad = 1;
            else atomicAdd(&tcnt[t], 1);
        }
        __syncthreads();
        for (int t = tid; t < T; t += 1024) {
            if (tcnt[t] != K) bad = 1;
            tcnt[t] = 0;
        }
    }
    __syncthreads();
    if (bad) {
        for (int i = tid; i < T * K; i += 1024) pl.pos[i] = -1;
        if (tid == 0) {
            *pl.n_seg = 0;
            *pl.n_sh_seg = 0;
            *pl.n_valid = 0;
            __hip_atomic_fetch_or(pl.err, kWsBuckets, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;  // uniform
    }
    if (tid == 0) *pl.n_valid = ep[E];
    // Segments are numbered heaviest first (the grouped GEMVs hand them out
    // in that order, so the last items left are the light ones): every
    // expert's full segments of kSegTok tokens in expert order, then the
    // experts' last partial segments by size, kSegTok-1 tokens down to 1.
    for (int e = tid; e < E; e += 1024) {
        const int g = ep[e + 1] - ep[e];
        nfull[e] = g / kSegTok;
        if (g % kSegTok) atomicAdd(&ccount[g % kSegTok], 1);
    }
    __syncthreads();
    const int n_sh = (T_sh + kSegTok - 1) / kSegTok;
    const int n_full = n_sh + block_exclusive_scan(nfull, fstart, tmp, E);
    for (int e = tid; e < E; e += 1024) fstart[e] += n_sh;
    if (tid == 0) {
        *pl.n_sh_seg = n_sh;
        int base = n_full;
        for (int c = kSegTok - 1; c >= 1; --c) {
            ccursor[c] = base;
            base += ccount[c];
        }
        *pl.n_seg = base;
        // the grouped GEMVs take work from these with device-scope atomics
        __hip_atomic_store(pl.ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pl.ctr + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    for (int e = tid; e < E && segs; e += 1024) {
        const int g = ep[e + 1] - ep[e], c = g % kSegTok;
        // order among equal-size partial segments is free: no result depends on it
        pid[e] = c ? atomicAdd(&ccursor[c], 1) : -1;
        for (int j = 0; j < nfull[e]; ++j) {
            const int sg = fstart[e] + j;
            pl.seg_e[sg] = e;
            pl.seg_p0[sg] = ep[e] + j * kSegTok;
            pl.seg_n[sg] = kSegTok;
        }
        if (c) {
            pl.seg_e[pid[e]] = e;
            pl.seg_p0[pid[e]] = ep[e] + nfull[e] * kSegTok;
            pl.seg_n[pid[e]] = c;
        }
    }
    const int N = ep[E];
    for (int j = tid; j < n_sh && segs; j += 1024) {
        pl.seg_e[j] = E;  // the shared expert
        pl.seg_p0[j] = N + j * kSegTok;
        pl.seg_n[j] = min(kSegTok, T_sh - j * kSegTok);
    }
    for (int t = tid; t < T_sh && segs; t += 1024) {
        pl.seg_of[N + t] = t / kSegTok;
        pl.idx_of[N + t] = t % kSegTok;
        pl.slot_tok[N + t] = t;
    }
    __syncthreads();
    for (int p = tid; p < N && segs; p += 1024) {
        int lo = 0, hi = E;  // largest e with ep[e] <= p
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (ep[mid] <= p) lo = mid; else hi = mid;
        }
        while (lo < E - 1 && ep[lo + 1] <= p) ++lo;  // skip empty buckets
        const int r = p - ep[lo], j = r / kSegTok;
        pl.seg_of[p] = j < nfull[lo] ? fstart[lo] + j : pid[lo];
        pl.idx_of[p] = r % kSegTok;
        pl.slot_tok[p] = tok[p];
    }
    // each token's slots in bucket order = expert order: every slot appends
    // itself to its token's (unordered) list in pos_buf, then takes the place
    // of its rank in that list
    for (int p = tid; p < N; p += 1024) {
        const int t = tok[p];
        if (t >= 0 && t < T) {
            const int c = atomicAdd(&tcnt[t], 1);
            if (c < K) pos_buf[(size_t)t * K + c] = p;
        }
    }
    __threadfence_block();
    __syncthreads();
    for (int p = tid; p < N; p += 1024) {
        const int t = tok[p];
        if (t >= 0 && t < T) {
            const int n = min(tcnt[t], K);
            int r = 0;
            for (int c = 0; c < n; ++c) r += pos_buf[(size_t)t * K + c] < p;
            pl.pos[(size_t)t * K + r] = p;
        }
    }
}

__global__ __launch_bounds__(1024) void k_moe_plan(const int* __restrict__ eptr, const int* __restrict__ tok,
                                                   int T, int E, int K, MoePlan pl) {
    plan_body(eptr, tok, T, E, K, 0, pl, pl.pos_tmp);
}


// ---------------------------------------------------------------------------
// Activation gather / SwiGLU into per-segment prepared activations

// Lane-major prepared activation of one segment (see load_record): token t
// of n_tok, block b, register image a, slice beta, hi (hl = 0) or lo part.
__device__ __forceinline__ size_t act_off(int n_tok, int b, int t, int a, int beta, int hl) {
    const int p = t >> 1;
    const bool half_pair = (n_tok & 1) && (p == (n_tok >> 1));
    const size_t base = (size_t)b * n_tok * 1024 + (size_t)p * 2048;
    if (half_pair) return base + (2 * beta + hl) * 32 + a * 8;
    return base + (4 * beta + 2 * (t & 1) + hl) * 32 + a * 8;
}

// One 256-element block's activation images, built by one wavefront (lane
// holds elements 4*lane .. 4*lane+3): the block's power-of-two scale from the
// wavefront maximum, fp16 hi and lo parts.
struct BlockImages {
    _Float16 hi[4], lo[4];
    int sc;
};
__device__ __forceinline__ BlockImages block_images(const float (&e)[4]) {
    BlockImages r;
    r.sc = pow2_scale_of_max(wave_max(fmaxf(fmaxf(fabsf(e[0]), fabsf(e[1])), fmaxf(fabsf(e[2]), fabsf(e[3])))));
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const float xs = ldexpf(e[c], r.sc);
        r.hi[c] = (_Float16)xs;
        r.lo[c] = (_Float16)(xs - (float)r.hi[c]);
    }
    return r;
}

// One wavefront per (slot p, block b). MODE 0: v = X[tok[p]]; MODE 1:
// v = silu(min(G[p],lim)) * clamp(U[p],-lim,lim), over the bucket slots and
// then the n_extra shared-expert slots.
template <int MODE>
__global__ __launch_bounds__(256) void k_prep_grouped(const float* __restrict__ X, const float* __restrict__ U,
                                                      const int* __restrict__ tok, const int* __restrict__ eptr,
                                                      int E, int nb, float lim, MoePlan pl,
                                                      uint8_t* __restrict__ act, size_t seg_stride, int n_extra) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + wave;
    const int N = *pl.n_valid + (*pl.n_seg > 0 ? n_extra : 0);
    if (item >= N * nb) return;
    const int p = item / nb, b = item - p * nb;
    const size_t row = MODE == 0 ? (size_t)tok[p] : (size_t)p;
    const size_t src = row * nb * 256 + (size_t)b * 256 + 4 * lane;
    const float4 v = *reinterpret_cast<const float4*>(X + src);
    float e[4] = {v.x, v.y, v.z, v.w};
    if (MODE == 1) {
        const float4 u = *reinterpret_cast<const float4*>(U + src);
        const float us[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            e[c] = swiglu1(e[c], us[c], lim);
        }
    }
    const BlockImages im = block_images(e);
    const int s = pl.seg_of[p], t = pl.idx_of[p], n = pl.seg_n[s];
    uint8_t* base = act + (size_t)s * seg_stride;
    const int a = lane >> 4, beta = lane & 15;
    *reinterpret_cast<u32x2_t*>(base + act_off(n, b, t, a, beta, 0)) = __builtin_bit_cast(u32x2_t, im.hi);
    *reinterpret_cast<u32x2_t*>(base + act_off(n, b, t, a, beta, 1)) = __builtin_bit_cast(u32x2_t, im.lo);
    if (lane == 0) reinterpret_cast<float*>(base + (size_t)nb * n * 1024)[(size_t)b * n + t] = ldexpf(1.0f, -im.sc);
}

// Per-token activation images of X (one 1 KiB image set per token and
// block, in the layout of a one-token segment, plus the block unscale):
// items (t, b) from `item0`, `n_waves` wavefronts in all.
__device__ __forceinline__ void token_images(const float* __restrict__ X, int T, int nb, uint8_t* __restrict__ timg,
                                             float* __restrict__ tus, int item0, int n_waves, uint32_t lane) {
    for (int item = item0; item < T * nb; item += n_waves) {
        const float4 v = *reinterpret_cast<const float4*>(X + (size_t)item * 256 + 4 * lane);
        const float e[4] = {v.x, v.y, v.z, v.w};
        const BlockImages im = block_images(e);
        const int a = lane >> 4, beta = lane & 15;
        uint8_t* base = timg + (size_t)item * 1024;
        *reinterpret_cast<u32x2_t*>(base + act_off(1, 0, 0, a, beta, 0)) = __builtin_bit_cast(u32x2_t, im.hi);
        *reinterpret_cast<u32x2_t*>(base + act_off(1, 0, 0, a, beta, 1)) = __builtin_bit_cast(u32x2_t, im.lo);
        if (lane == 0) tus[item] = ldexpf(1.0f, -im.sc);
    }
}

// The front of a whole routed step. The first n_rank workgroups rank the
// tokens (token t on workgroup t % n_rank, wavefront (t / n_rank) % 16) into
// asg_e / asg_w; the last of them to finish (a ticket in the plan's
// counters, reset again at the end) counts the assignments per expert,
// bucket-sorts them and makes the work plan (with T_sh shared-expert
// tokens), its data in LDS when T * K <= kRouteLdsAsg. The other workgroups
// build the per-token X images meanwhile.
template <int J, bool kLds>
__global__ __launch_bounds__(1024) void k_moe_front(const float* __restrict__ logits, int T, int E, int K, int mode,
                                                    const float* __restrict__ bias, float routed_scale,
                                                    int norm_topk, int* __restrict__ eptr, int* __restrict__ tok,
                                                    float* __restrict__ wt, int* __restrict__ sel,
                                                    int* __restrict__ asg_e, float* __restrict__ asg_w, int T_sh,
                                                    MoePlan pl, const float* __restrict__ X, int nb,
                                                    uint8_t* __restrict__ timg, float* __restrict__ tus,
                                                    int n_rank, int plan_segs) {
    __shared__ float rank_score[16][kMaxTopK];
    __shared__ int cnt[kMaxExperts];
    __shared__ int cursor[kMaxExperts];
    __shared__ __attribute__((aligned(16))) int chunk_e[1024];
    __shared__ int lds_e[kLds ? kRouteLdsAsg : 1];
    __shared__ float lds_w[kLds ? kRouteLdsAsg : 1];
    __shared__ int l_eptr[kLds ? kMaxExperts + 1 : 1], l_tok[kLds ? kRouteLdsAsg : 1], l_pos[kLds ? kRouteLdsAsg : 1];
    __shared__ uint32_t ticket_old;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int G = n_rank;
    if ((int)blockIdx.x >= G) {
        token_images(X, T, nb, timg, tus, ((int)blockIdx.x - G) * 16 + wave, ((int)gridDim.x - G) * 16, lane);
        return;
    }
    uint32_t* ticket = pl.ctr + 2;
    const int N = T * K;
    if (kLds && G == 1) {  // uniform
        // one ranking workgroup: the assignments and their counts go
        // straight to LDS, and no other workgroup has to see them
        for (int e = tid; e < E; e += 1024) cnt[e] = 0;
        __syncthreads();
        topk_loop<J>(logits, T, E, K, mode, bias, routed_scale, norm_topk, sel, lds_e, lds_w, cnt, rank_score, wave,
                     16, wave, lane);
        __syncthreads();
        bucket_body(T, E, K, eptr, tok, wt, lds_e, lds_w, cnt, cursor, chunk_e, l_eptr, l_tok);
        __syncthreads();
        plan_body(l_eptr, l_tok, T, E, K, T_sh, pl, l_pos, plan_segs != 0);
        return;
    }
    topk_loop<J>(logits, T, E, K, mode, bias, routed_scale, norm_topk, sel, asg_e, asg_w, nullptr, rank_score,
                 wave * G + blockIdx.x, G * 16, wave, lane);
    // every wavefront's stores, then one ticket per workgroup
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old >= (uint32_t)G) __hip_atomic_fetch_or(pl.err, kWsTicket, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ticket_old = old;
    }
    __syncthreads();
    if (ticket_old != (uint32_t)G - 1) return;  // uniform
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    for (int e = tid; e < E; e += 1024) cnt[e] = 0;
    __syncthreads();
    for (int a = tid; a < N; a += 1024) {
        const int e = asg_e[a];
        if constexpr (kLds) {
            lds_e[a] = e;
            lds_w[a] = asg_w[a];
        }
        atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if constexpr (kLds) {
        bucket_body(T, E, K, eptr, tok, wt, lds_e, lds_w, cnt, cursor, chunk_e, l_eptr, l_tok);
        __syncthreads();
        plan_body(l_eptr, l_tok, T, E, K, T_sh, pl, l_pos, plan_segs != 0);
    } else {
        bucket_body(T, E, K, eptr, tok, wt, asg_e, asg_w, cnt, cursor, chunk_e, nullptr, nullptr);
        // the plan reads eptr / tok as the bucket sort wrote them
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "agent");
        __syncthreads();
        plan_body(eptr, tok, T, E, K, T_sh, pl, pl.pos_tmp, plan_segs != 0);
    }
    if (tid == 0) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Ragged grouped GEMV

struct GroupedArgs {
    const uint8_t* w[2];      // T64 tensors holding every expert's rows
    const uint8_t* w_sh[2];   // the shared expert's T64 tensors (segments of expert n_exp), or null
    float* y[2];              // [N][rows_per_expert] per tensor, bucket order
    const uint8_t* act;       // per-segment prepared activations
    size_t seg_stride;
    int n_tensors;
    int nb;                   // blocks per row
    int tiles;                // 64-row tiles per expert
    int tiles_per_item;       // consecutive row tiles one work item streams (divides tiles)
    int rows;                 // rows per expert (= output width)
    MoePlan pl;
    int ctr_index;
    int n_exp;                // expert id of the shared expert's segments
    // gather mode: activations are per-token images (token_images), read
    // through the slots' tokens, instead of per-segment images
    const uint8_t* timg;
    const float* tus;
};

// load_record with the activation gathered from per-token images: lane L of
// pair p reads its 32 bytes from the image set of token 2p + ((L >> 1) & 1)
// (token 2p for a last pair holding one token) at byte offset toff[p] of
// timg_b, the images of block b.
template <int NP>
__device__ __forceinline__ void load_record_gather(Rec<NP>& r, const uint8_t* rec, const uint8_t* timg_b,
                                                   const size_t (&toff)[NP], uint32_t lane) {
    // the record non-temporal, as in load_record
#pragma unroll
    for (int i = 0; i < 6; ++i)
        r.u[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(rec + i * kUnitBytes + lane * 16u));
    r.d = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(rec + kRecordDOffset + lane * 2u));
    const uint32_t slot_half = (lane >> 2) * 2 + (lane & 1);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const uint8_t* src = timg_b + toff[p] + slot_half * 32u;
        const u32x4_t v0 = *reinterpret_cast<const u32x4_t*>(src);
        const u32x4_t v1 = *reinterpret_cast<const u32x4_t*>(src + 16);
        r.a[p][0] = u32x2_t{v0.x, v0.y};
        r.a[p][1] = u32x2_t{v0.z, v0.w};
        r.a[p][2] = u32x2_t{v1.x, v1.y};
        r.a[p][3] = u32x2_t{v1.z, v1.w};
    }
}

// One (segment, tensor, tile) item: the wavefront walks the tile's nb
// records through a 2-deep ring and writes the 64 rows x n tokens result.
// nt consecutive row tiles (records rec0 .. rec0 + nt*nb - 1, tile-major) of
// one segment: the ring runs on across the tile boundaries; each tile's sums
// go to y at its end.
// kGather: the activations come from per-token images (timg, tus) through
// slot_tok[p0 ..], not from the segment's own images at act.
template <int NP, bool kGather>
__device__ __forceinline__ void grouped_tile(const uint8_t* tbl, uint32_t lb, uint32_t lane, const uint8_t* rec0,
                                             const uint8_t* act, int n, int nb, int nt, float* y, int rows,
                                             int row0, const uint8_t* timg, const float* tus,
                                             const int* slot_tok, int p0) {
    // records in flight: two, or one for four token pairs (a record and its
    // activation images take 58 registers there; two of them spilled)
    constexpr int PF = NP >= 4 ? 1 : 2;
    const int nrec = nt * nb;
    const float* xsc = reinterpret_cast<const float*>(act + (size_t)nb * n * 1024);
    // The block unscales travel with the record ring: one wait per record
    // covers both, where a load issued at the product would expose its
    // latency.
    Rec<NP> ring[PF];
    const int tl = min((int)(lane & 7u), n - 1);
    size_t toff[NP];
    size_t us_row = 0;
    if constexpr (kGather) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const bool half = (p == NP - 1) && (n & 1);
            const int tt = min(2 * p + (half ? 0 : (int)((lane >> 1) & 1u)), n - 1);
            toff[p] = (size_t)slot_tok[p0 + tt] * nb * 1024;
        }
        us_row = (size_t)slot_tok[p0 + tl] * nb;
    }
    auto fill = [&](Rec<NP>& r, int k) {  // record k of the item (clamped to the last)
        k = min(k, nrec - 1);
        const int b = k % nb;
        if constexpr (kGather) {
            load_record_gather<NP>(r, rec0 + (size_t)k * kRecordBytes, timg + (size_t)b * 1024, toff, lane);
            r.xs = __builtin_bit_cast(uint32_t, tus[us_row + b]);
        } else {
            load_record<NP>(r, rec0 + (size_t)k * kRecordBytes, act + (size_t)b * n * 1024, lane, n);
            r.xs = __builtin_bit_cast(uint32_t, xsc[(size_t)b * n + tl]);
        }
    };
#pragma unroll
    for (int s = 0; s < PF; ++s) {
        fill(ring[s], s);
        // slot order kept, so the loop's first wait covers slot 0 only
        __builtin_amdgcn_sched_barrier(0);
    }
    float acc[2 * NP];
#pragma unroll
    for (int t = 0; t < 2 * NP; ++t) acc[t] = 0.0f;
    int kb = 0, tile = 0;  // block within the tile, tile within the item
    for (int k0 = 0; k0 < nrec; k0 += PF) {
#pragma unroll
        for (int s = 0; s < PF; ++s) {
            const int k = k0 + s;
            if (k < nrec) {
                float blk[2 * NP];
#pragma unroll
                for (int t = 0; t < 2 * NP; ++t) blk[t] = 0.0f;
                record_dot<NP>(tbl, ring[s], lb, blk);
                const float d4 = (float)__builtin_bit_cast(_Float16, (uint16_t)ring[s].d) * 0.25f;
                // an infinite or NaN d makes the row NaN, as the reference's
                // sum of that block's +-inf products of both signs does
                const float dz = d4 - d4;
#pragma unroll
                for (int t = 0; t < 2 * NP; ++t)
                    if (t < n) acc[t] = fmaf(d4 * rec_unscale(ring[s], t), blk[t], acc[t] + dz);
                if (++kb == nb) {  // uniform
#pragma unroll
                    for (int t = 0; t < 2 * NP; ++t) {
                        if (t < n) y[(size_t)t * rows + row0 + tile * kTileRows + lane] = acc[t];
                        acc[t] = 0.0f;
                    }
                    kb = 0;
                    ++tile;
                }
            }
            fill(ring[s], k + PF);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

constexpr int kGroupedThreads = 256;

__global__ __launch_bounds__(kGroupedThreads, 2) void k_gemv_grouped(GroupedArgs g) {
    __shared__ __attribute__((aligned(16))) uint8_t tbl[kGridTableBytes];
    const int tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t lb = (lane & 31u) << 3;
    GridWords<kGroupedThreads> gw;
    grid_words<kGroupedThreads>(gw, tid);
    grid_table_store<kGroupedThreads>(tbl, gw, tid);
    lds_barrier();
    const int groups = g.tiles / g.tiles_per_item;  // items per segment and tensor
    const int per_seg = g.n_tensors * groups;
    const int n_items = *g.pl.n_seg * per_seg;
    // the first round is static (wavefront i takes item i), the rest come
    // from the counter: 2048 wavefronts taking tickets on one address at
    // once serialise for tens of microseconds
    constexpr int kWavesPerGroup = kGroupedThreads / 64;
    const uint32_t n_waves = gridDim.x * kWavesPerGroup;
    uint32_t item = blockIdx.x * kWavesPerGroup + (tid >> 6);
    while (true) {
        if (item >= (uint32_t)n_items) break;
        const int s = item / per_seg;
        const int rem = item - s * per_seg;
        const int ten = rem / groups, tile = (rem - ten * groups) * g.tiles_per_item;
        const int e = g.pl.seg_e[s], p0 = g.pl.seg_p0[s], n = g.pl.seg_n[s];
        const uint8_t* rec0 = e == g.n_exp ? g.w_sh[ten] + (size_t)tile * g.nb * kRecordBytes
                                           : g.w[ten] + ((size_t)e * g.tiles + tile) * g.nb * kRecordBytes;
        const uint8_t* act = g.act + (size_t)s * g.seg_stride;
        float* y = g.y[ten] + (size_t)p0 * g.rows;
        const int nt = g.tiles_per_item;
#define GPEED_GROUPED_TILE(NP)                                                                                   \
    (g.timg ? grouped_tile<NP, true>(tbl, lb, lane, rec0, act, n, g.nb, nt, y, g.rows, tile * kTileRows, g.timg, \
                                     g.tus, g.pl.slot_tok, p0)                                                   \
            : grouped_tile<NP, false>(tbl, lb, lane, rec0, act, n, g.nb, nt, y, g.rows, tile * kTileRows,       \
                                      nullptr, nullptr, nullptr, 0))
        switch ((n + 1) >> 1) {
            case 1: GPEED_GROUPED_TILE(1); break;
            case 2: GPEED_GROUPED_TILE(2); break;
            case 3: GPEED_GROUPED_TILE(3); break;
            default: GPEED_GROUPED_TILE(4); break;
        }
#undef GPEED_GROUPED_TILE
        uint32_t t = 0;
        if (lane == 0) t = __hip_atomic_fetch_add(g.pl.ctr + g.ctr_index, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        item = n_waves + __builtin_amdgcn_readfirstlane(__shfl(t, 0));
    }
}

// ---------------------------------------------------------------------------
// Weighted combine (model_batch.cpp:257-261): Y[t] = sum_k wt * D[slot],
// slots in expert order, one fma per term.
// With the shared expert (sh: its down rows, one per token; model_batch.cpp:
// 264-280), Y[t] = that sum + sh[t] (add_f32), unless the plan rejected
// the buckets (n_seg 0).
__global__ __launch_bounds__(256) void k_moe_combine(const float* __restrict__ D, const float* __restrict__ wt,
                                                     const int* __restrict__ pos, int T, int K, int H,
                                                     float* __restrict__ Y, const float* __restrict__ sh,
                                                     const int* __restrict__ n_seg) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t n4 = (size_t)T * H / 4;
    if (i >= n4) return;
    const int t = (int)(i * 4 / H);
    const int h = (int)(i * 4 - (size_t)t * H);
    float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int k = 0; k < K; ++k) {
        const int p = pos[(size_t)t * K + k];
        if (p < 0) continue;  // buckets rejected by the plan
        const float w = wt[p];
        const float4 d = *reinterpret_cast<const float4*>(D + (size_t)p * H + h);
        y.x = fmaf(w, d.x, y.x);
        y.y = fmaf(w, d.y, y.y);
        y.z = fmaf(w, d.z, y.z);
        y.w = fmaf(w, d.w, y.w);
    }
    if (sh && *n_seg > 0) {
        const float4 d = *reinterpret_cast<const float4*>(sh + (size_t)t * H + h);
        y.x = y.x + d.x;
        y.y = y.y + d.y;
        y.z = y.z + d.z;
        y.w = y.w + d.w;
    }
    *reinterpret_cast<float4*>(Y + (size_t)t * H + h) = y;
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

struct MoeLayout {
    size_t plan_off[10];
    size_t act1, g, u, act2, d, total;
    size_t eptr, tok, wt, sel, asg_e, asg_w, timg, tus;  // the whole-step path only
    size_t xg, xg_uns, gtiles, gcount, hg, hg_uns, sh1, sh2;  // its grouped-GEMM form only
    size_t stride1, stride2;
    int seg_max;
};

// The whole step runs its experts as grouped GEMMs (each expert's weights
// read once per 64 of its tokens) where the buckets average at least this
// many tokens, and as grouped GEMVs over 8-token segments below (the GEMV
// streams the weights once per segment). The same crossover as matmul_quant:
// from 9 tokens one GEMM pass beats two GEMV passes.
constexpr int kMoeGemmMinAvg = 9;
bool moe_use_gemm(int T, int E, int K) { return (long long)T * K >= (long long)kMoeGemmMinAvg * E; }

// T_sh: shared-expert tokens (0 or T). fused: the whole step from the
// logits (router outputs, router scratch and per-token X images in the
// workspace, no per-segment X images).
MoeLayout moe_layout(int T, int E, int K, int H, int I, int T_sh = 0, bool fused = false) {
    MoeLayout L{};
    const size_t N = (size_t)T * K, NS = N + (size_t)T_sh;
    L.seg_max = (int)((N + (size_t)(kSegTok - 1) * E) / kSegTok + 1) + (T_sh + kSegTok - 1) / kSegTok;
    size_t off = kWsHeader;
    const size_t sizes[10] = {256, 4 * (size_t)L.seg_max, 4 * (size_t)L.seg_max, 4 * (size_t)L.seg_max,
                              4 * NS, 4 * NS, 4 * N, 256, 4 * NS, 4 * N};
    for (int i = 0; i < 10; ++i) {
        L.plan_off[i] = off;
        off += align256(sizes[i]);
    }
    L.stride1 = align256((size_t)(H / kQK) * kSegTok * (1024 + 4));
    L.stride2 = align256((size_t)(I / kQK) * kSegTok * (1024 + 4));
    if (fused) {
        L.eptr = off; off += align256(4 * ((size_t)E + 1));
        L.tok = off; off += align256(4 * N);
        L.wt = off; off += align256(4 * N);
        L.sel = off; off += align256(4 * N);
        L.asg_e = off; off += align256(4 * N);
        L.asg_w = off; off += align256(4 * N);
        L.timg = off; off += (size_t)T * (H / kQK) * 1024;
        L.tus = off; off += align256((size_t)T * (H / kQK) * 4);
    } else {
        L.act1 = off; off += L.stride1 * L.seg_max;
    }
    L.g = off; off += align256(NS * I * 4);
    L.u = off; off += align256(NS * I * 4);
    L.act2 = off; off += L.stride2 * L.seg_max;
    L.d = off; off += align256(NS * H * 4);
    L.total = off;
    return L;
}

// The grouped-GEMM form runs the shared expert's T_sh tokens as one more
// bucket of its grouped launches where its gate/up GEMM alone (fp32 X,
// 64-token tiles, 256-row tiles of gate and up) would not give every CU a
// tile of the 32x32 form: merged, its tiles fill the grouped launches' last
// round (256 tokens 717 -> 682 us, 128 tokens 569 -> 511 us on one box);
// at 1024 tokens the separate 32x32 GEMMs win (1883 against 1971 us).
bool moe_merge_shared(int T_sh, int I, int num_cus) {
    const long long tiles = (long long)((T_sh + 63) / 64) * 2 * ((I + 255) / 256);
    return T_sh > 0 && tiles < (num_cus > 0 ? num_cus : 256);
}

// The grouped-GEMM form of the whole step: the layout above (its segment
// images unused) and, after it, the per-token X images, the expert tile
// table, the slot-ordered SwiGLU images and the shared expert's GEMM
// workspaces.
MoeLayout moe_gemm_layout(int T, int E, int K, int H, int I, int T_sh, int num_cus) {
    MoeLayout L = moe_layout(T, E, K, H, I, T_sh, true);
    const size_t S = (size_t)T * K;
    size_t off = L.total;
    L.xg = off; off += align256(2 * (size_t)T * H * 2);
    L.xg_uns = off; off += align256((size_t)T * 4);
    const bool merge = moe_merge_shared(T_sh, I, num_cus);
    const size_t NS = S + (size_t)(merge ? T_sh : 0);
    L.gtiles = off; off += align256(4 * (size_t)grp_tiles_cap((int)NS, E + 1, 0));
    L.gcount = off; off += 256;
    L.hg = off; off += align256(2 * NS * I * 2);
    L.hg_uns = off; off += align256(NS * 4);
    if (T_sh && !merge) {
        L.sh1 = off; off += align256(gemm2_ws_bytes(T_sh, I, I, H, 0, num_cus));
        L.sh2 = off; off += align256(gemm_ws_bytes(T_sh, H, I, 0, num_cus));
    }
    L.total = off;
    return L;
}

MoePlan plan_ptrs(uint8_t* ws, const MoeLayout& L) {
    MoePlan p;
    p.n_seg = reinterpret_cast<int*>(ws + L.plan_off[0]);
    p.n_valid = p.n_seg + 1;
    p.n_sh_seg = p.n_seg + 2;
    p.slot_tok = reinterpret_cast<int*>(ws + L.plan_off[8]);
    p.pos_tmp = reinterpret_cast<int*>(ws + L.plan_off[9]);
    p.err = reinterpret_cast<uint32_t*>(ws);
    p.ctr = reinterpret_cast<uint32_t*>(ws + L.plan_off[7]);
    p.seg_e = reinterpret_cast<int*>(ws + L.plan_off[1]);
    p.seg_p0 = reinterpret_cast<int*>(ws + L.plan_off[2]);
    p.seg_n = reinterpret_cast<int*>(ws + L.plan_off[3]);
    p.seg_of = reinterpret_cast<int*>(ws + L.plan_off[4]);
    p.idx_of = reinterpret_cast<int*>(ws + L.plan_off[5]);
    p.pos = reinterpret_cast<int*>(ws + L.plan_off[6]);
    return p;
}

}  // namespace

size_t moe_route_ws_bytes(int T, int K) { return 2 * align256((size_t)T * K * 4); }

hipError_t launch_moe_route(const float* logits, int T, int E, int K, int mode, const float* bias,
                            float routed_scale, int norm_topk, int* eptr, int* tok, float* wt, int* sel,
                            uint8_t* ws, hipStream_t s) {
    int* asg_e = reinterpret_cast<int*>(ws);
    float* asg_w = reinterpret_cast<float*>(ws + align256((size_t)T * K * 4));
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3(1), dim3(1024), 0, s, logits, T, E, K, mode, bias, routed_scale, norm_topk,
                           eptr, tok, wt, sel, asg_e, asg_w);
    };
    const bool lds = (long long)T * K <= kRouteLdsAsg;
    if (E <= 64) lds ? go(k_moe_route<1, true>) : go(k_moe_route<1, false>);
    else if (E <= 128) lds ? go(k_moe_route<2, true>) : go(k_moe_route<2, false>);
    else if (E <= 256) lds ? go(k_moe_route<4, true>) : go(k_moe_route<4, false>);
    else lds ? go(k_moe_route<kMaxExperts / 64, true>) : go(k_moe_route<kMaxExperts / 64, false>);
    return hipGetLastError();
}

size_t moe_ws_bytes(int T, int E, int K, int H, int I) { return moe_layout(T, E, K, H, I).total; }

hipError_t launch_moe_experts(const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down, int E, int H,
                              int I, const float* X, int T, int K, const int* eptr, const int* tok,
                              const float* wt, float lim, float* Y, uint8_t* ws, int num_cus, hipStream_t s) {
    const MoeLayout L = moe_layout(T, E, K, H, I);
    const MoePlan pl = plan_ptrs(ws, L);
    const int N = T * K;
    const int nbH = H / kQK, nbI = I / kQK;
    float* G = reinterpret_cast<float*>(ws + L.g);
    float* U = reinterpret_cast<float*>(ws + L.u);
    float* D = reinterpret_cast<float*>(ws + L.d);
    hipLaunchKernelGGL(k_moe_plan, dim3(1), dim3(1024), 0, s, eptr, tok, T, E, K, pl);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_prep_grouped<0>, dim3((N * nbH + 3) / 4), dim3(256), 0, s, X, nullptr, tok, eptr, E,
                       nbH, 0.0f, pl, ws + L.act1, L.stride1, 0);
    const int grid = (num_cus > 0 ? num_cus : 256) * 2;
    GroupedArgs ga{};
    ga.w[0] = w_gate;
    ga.w[1] = w_up;
    ga.y[0] = G;
    ga.y[1] = U;
    ga.act = ws + L.act1;
    ga.seg_stride = L.stride1;
    ga.n_tensors = 2;
    ga.nb = nbH;
    ga.tiles = I / kTileRows;
    ga.tiles_per_item = 1;
    ga.rows = I;
    ga.pl = pl;
    ga.ctr_index = 0;
    ga.n_exp = E;
    e = launch_timed(kProfGrouped, k_gemv_grouped, dim3(grid), dim3(kGroupedThreads), 0, s, ga);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_prep_grouped<1>, dim3((N * nbI + 3) / 4), dim3(256), 0, s, G, U, tok, eptr, E, nbI,
                       lim, pl, ws + L.act2, L.stride2, 0);
    GroupedArgs gd = ga;
    gd.w[0] = w_down;
    gd.w[1] = w_down;
    gd.y[0] = D;
    gd.y[1] = D;
    gd.act = ws + L.act2;
    gd.seg_stride = L.stride2;
    gd.n_tensors = 1;
    gd.nb = nbI;
    gd.tiles = H / kTileRows;
    // short rows (few blocks per tile) take several tiles per item, so the
    // ring's start-up is paid once per ~16 records
    gd.tiles_per_item = 1;
    while (gd.tiles_per_item < 4 && gd.tiles % (2 * gd.tiles_per_item) == 0 && gd.nb * gd.tiles_per_item < 16)
        gd.tiles_per_item *= 2;
    gd.rows = H;
    gd.ctr_index = 1;
    e = launch_timed(kProfGrouped, k_gemv_grouped, dim3(grid), dim3(kGroupedThreads), 0, s, gd);
    if (e != hipSuccess) return e;
    const size_t n4 = (size_t)T * H / 4;
    hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, D, wt, pl.pos, T, K, H,
                       Y, nullptr, pl.n_seg);
    return hipGetLastError();
}

size_t moe_batch_ws_bytes(int T, int E, int K, int H, int I, int shared, int num_cus) {
    if (moe_use_gemm(T, E, K)) return moe_gemm_layout(T, E, K, H, I, shared ? T : 0, num_cus).total;
    return moe_layout(T, E, K, H, I, shared ? T : 0, true).total;
}

hipError_t launch_moe_batch(const float* logits, int T, int E, int K, int mode, const float* bias,
                            float routed_scale, int norm_topk, const uint8_t* w_gate, const uint8_t* w_up,
                            const uint8_t* w_down, const uint8_t* w_gate_sh, const uint8_t* w_up_sh,
                            const uint8_t* w_down_sh, int H, int I, const float* X, float lim, float* Y,
                            int* eptr_out, int* tok_out, float* wt_out, uint8_t* ws, int num_cus, hipStream_t s) {
    const int T_sh = w_gate_sh ? T : 0;
    const bool gemm = moe_use_gemm(T, E, K);
    const MoeLayout L = gemm ? moe_gemm_layout(T, E, K, H, I, T_sh, num_cus) : moe_layout(T, E, K, H, I, T_sh, true);
    const MoePlan pl = plan_ptrs(ws, L);
    const int N = T * K, NS = N + T_sh;
    const int nbH = H / kQK, nbI = I / kQK;
    int* eptr = eptr_out ? eptr_out : reinterpret_cast<int*>(ws + L.eptr);
    int* tok = tok_out ? tok_out : reinterpret_cast<int*>(ws + L.tok);
    float* wt = wt_out ? wt_out : reinterpret_cast<float*>(ws + L.wt);
    float* G = reinterpret_cast<float*>(ws + L.g);
    float* U = reinterpret_cast<float*>(ws + L.u);
    float* D = reinterpret_cast<float*>(ws + L.d);
    uint8_t* timg = ws + L.timg;
    float* tus = reinterpret_cast<float*>(ws + L.tus);
    // 1. router, per-token X images, bucket sort and work plan
    // ranking workgroups: one token per wavefront up to 64 of them; image
    // workgroups: one (token, block) item per wavefront up to 192
    // (the grouped-GEMM form gathers its own images: no image workgroups)
    // (up to 32 tokens: one ranking workgroup, two tokens per wavefront,
    // whose assignments stay in its LDS)
    const int n_rank = T <= 32 ? 1 : std::min((T + 15) / 16, 64);
    const int groups = n_rank + (gemm ? 0 : std::min((T * nbH + 15) / 16, 192));
    // (the grouped-GEMM form runs the shared expert as GEMMs of its own, so
    // its plan holds the routed segments only)
    const int T_plan = gemm ? 0 : T_sh;
    auto front = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3(groups), dim3(1024), 0, s, logits, T, E, K, mode, bias, routed_scale,
                           norm_topk, eptr, tok, wt, reinterpret_cast<int*>(ws + L.sel),
                           reinterpret_cast<int*>(ws + L.asg_e), reinterpret_cast<float*>(ws + L.asg_w), T_plan, pl, X,
                           nbH, timg, tus, n_rank, gemm ? 0 : 1);
    };
    const bool lds = (long long)T * K <= kRouteLdsAsg;
    if (E <= 64) lds ? front(k_moe_front<1, true>) : front(k_moe_front<1, false>);
    else if (E <= 128) lds ? front(k_moe_front<2, true>) : front(k_moe_front<2, false>);
    else if (E <= 256) lds ? front(k_moe_front<4, true>) : front(k_moe_front<4, false>);
    else lds ? front(k_moe_front<kMaxExperts / 64, true>) : front(k_moe_front<kMaxExperts / 64, false>);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (gemm) {
        // prefill-sized batches (model_batch.cpp:224-280 at run_chunk's n,
        // model_batch.cpp:391): X gathered into the slots' GEMM images, each
        // expert's gate and up as grouped GEMMs over its bucket (row0 = e*I),
        // SwiGLU images, the grouped down GEMM (row0 = e*H), the shared
        // expert as the dense MLP's GEMMs over every token, then the combine
        uint32_t* err = reinterpret_cast<uint32_t*>(ws);
        _Float16* xg = reinterpret_cast<_Float16*>(ws + L.xg);
        float* xg_uns = reinterpret_cast<float*>(ws + L.xg_uns);
        int* gtiles = reinterpret_cast<int*>(ws + L.gtiles);
        int* gcount = reinterpret_cast<int*>(ws + L.gcount);
        _Float16* hg = reinterpret_cast<_Float16*>(ws + L.hg);
        float* hg_uns = reinterpret_cast<float*>(ws + L.hg_uns);
        // X's images once per token; the gate/up GEMM reads a slot's row
        // through its token
        e = launch_prep_x_rows(T, H, s, X, nullptr, 0.0f, xg, xg_uns, nullptr);
        // the shared expert joins the grouped launches as one more bucket
        // (expert id E, slots N .. N + T_sh - 1, its own tensors), unless
        // its gate/up GEMM alone fills the CUs with 32x32 tiles
        const int T_m = moe_merge_shared(T_sh, I, num_cus) ? T_sh : 0;
        const int NM = N + T_m;
        const int mt = grp_tile_mt(N, E);
        if (e == hipSuccess) e = launch_grp_tiles(eptr, E, N, mt, gtiles, gcount, s, T_m);
        if (e == hipSuccess)
            e = launch_gemm_grouped(w_gate, w_up, I, H, E, eptr, NM, xg, xg_uns, G, U, gtiles, gcount, err, s, mt, tok,
                                    T, w_gate_sh, w_up_sh, T_m);
        if (e == hipSuccess) e = launch_prep_x_rows(NM, I, s, G, U, lim, hg, hg_uns, nullptr);
        if (e == hipSuccess)
            e = launch_gemm_grouped(w_down, nullptr, H, I, E, eptr, NM, hg, hg_uns, D, nullptr, gtiles, gcount, err,
                                    s, mt, nullptr, 0, w_down_sh, nullptr, T_m);
        if (e == hipSuccess && T_sh && !T_m) {
            float* Gs = G + (size_t)N * I;
            float* Us = U + (size_t)N * I;
            e = launch_gemm2(w_gate_sh, 0, I, w_up_sh, 0, I, H, X, 0, T, Gs, Us, ws + L.sh1, err, num_cus, s);
            if (e == hipSuccess)
                e = launch_gemm(w_down_sh, 0, I, H, Gs, 0, T, D + (size_t)N * H, ws + L.sh2, err, num_cus, s, Us, lim);
        }
        if (e != hipSuccess) return e;
        const size_t n4 = (size_t)T * H / 4;
        hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, D, wt, pl.pos, T, K,
                           H, Y, T_sh ? D + (size_t)N * H : nullptr, pl.n_seg);
        return hipGetLastError();
    }
    // 2. gate / up of every segment (the shared expert's first)
    const int grid = (num_cus > 0 ? num_cus : 256) * 2;
    GroupedArgs ga{};
    ga.w[0] = w_gate;
    ga.w[1] = w_up;
    ga.w_sh[0] = w_gate_sh;
    ga.w_sh[1] = w_up_sh;
    ga.y[0] = G;
    ga.y[1] = U;
    ga.act = nullptr;
    ga.timg = timg;
    ga.tus = tus;
    ga.n_tensors = 2;
    ga.nb = nbH;
    ga.tiles = I / kTileRows;
    ga.tiles_per_item = 1;
    ga.rows = I;
    ga.pl = pl;
    ga.ctr_index = 0;
    ga.n_exp = E;
    e = launch_timed(kProfGrouped, k_gemv_grouped, dim3(grid), dim3(kGroupedThreads), 0, s, ga);
    if (e != hipSuccess) return e;
    // 3. SwiGLU images per slot
    hipLaunchKernelGGL(k_prep_grouped<1>, dim3((NS * nbI + 3) / 4), dim3(256), 0, s, G, U, tok, eptr, E, nbI, lim,
                       pl, ws + L.act2, L.stride2, T_sh);
    // 4. down
    GroupedArgs gd = ga;
    gd.w[0] = w_down;
    gd.w[1] = w_down;
    gd.w_sh[0] = w_down_sh;
    gd.w_sh[1] = w_down_sh;
    gd.y[0] = D;
    gd.y[1] = D;
    gd.act = ws + L.act2;
    gd.seg_stride = L.stride2;
    gd.timg = nullptr;
    gd.tus = nullptr;
    gd.n_tensors = 1;
    gd.nb = nbI;
    gd.tiles = H / kTileRows;
    gd.tiles_per_item = 1;
    while (gd.tiles_per_item < 4 && gd.tiles % (2 * gd.tiles_per_item) == 0 && gd.nb * gd.tiles_per_item < 16)
        gd.tiles_per_item *= 2;
    gd.rows = H;
    gd.ctr_index = 1;
    e = launch_timed(kProfGrouped, k_gemv_grouped, dim3(grid), dim3(kGroupedThreads), 0, s, gd);
    if (e != hipSuccess) return e;
    // 5. weighted combine in expert order, then the shared expert's rows
    const size_t n4 = (size_t)T * H / 4;
    hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, D, wt, pl.pos, T, K, H,
                       Y, T_sh ? D + (size_t)N * H : nullptr, pl.n_seg);
    return hipGetLastError();
}

}  // namespace gpeed
