// SPDX-License-Identifier: MIT
//
// Backward kernels of libdbs_hip for gfx950: the surrogate gradient of the
// decode's score outputs (each output differentiated along its own path with
// the selection held fixed) and the backtrack of the final beams.
//
//  * path_walk: one workgroup per example (one wavefront for K <= 64) walks
//    the trace from its last step and produces, per selected slot, the
//    gradient of the log-prob entry it used ("draws"). Per step every slot's draw is formed in the reference's
//    operation order and each parent sums its children in slot order
//    (reference src/decoder.cpp:565-624, 668-683).
//  * dense_gradient: one workgroup per [V] row writes the row's gradient once.
//    From logits, a row with entries g gets g_v - softmax(x_v) * S with S the
//    entries summed in token order (reference src/decoder.hpp:212-242);
//    otherwise only the entries are non-zero. The fresh mode stores 0 + value
//    in float32, float16 or bfloat16, so no zero-fill pass and no cast pass
//    are needed; the accumulate mode adds into a float32 buffer.
#include <hip/hip_runtime.h>

#include "dbs_cuda.h"
#include "engine.hpp"
#include "row_helpers.hpp"

namespace dbs_hip {

namespace {

constexpr int kWalkThreads = 256;
constexpr int kDenseThreads = 256;
constexpr int kDenseBatch = 8;  // 16-byte logits loads in flight per thread (dense gradient)

__global__ __launch_bounds__(kWalkThreads) void path_walk_kernel(BackwardParams p) {
    __shared__ float s_sum0[DBS_CUDA_MAX_BEAM];
    __shared__ float s_sum1[DBS_CUDA_MAX_BEAM];
    float* next = s_sum0;  // incoming gradient of each slot from the later steps
    float* prev = s_sum1;
    __shared__ float draw[DBS_CUDA_MAX_BEAM];
    __shared__ int32_t par[DBS_CUDA_MAX_BEAM];
    const int b = static_cast<int>(blockIdx.x);
    const int tid = static_cast<int>(threadIdx.x);
    const int K = p.K, T = p.T, V = p.V;
    const int steps_b = p.steps ? p.steps[b] : T;
    const int Kb = p.beams ? p.beams[b] : K;  // slots past the example's beams carry nothing
    for (int k = tid; k < K; k += kWalkThreads) next[k] = 0.0f;
    // steps the example did not decode carry no gradient
    for (int64_t i = static_cast<int64_t>(steps_b) * K + tid; i < static_cast<int64_t>(T) * K; i += kWalkThreads)
        p.draws[static_cast<int64_t>(b) * T * K + i] = 0.0f;
    __syncthreads();
    // A slot's trace entries and incoming gradients do not depend on the walk,
    // so with one slot per thread (K <= kWalkThreads) step t - 1's are loaded
    // into registers while step t is walked: the loop waits on the barriers,
    // not on a memory round trip per step.
    struct SlotIn {
        int parent = -1, len = 0, tok = -1;
        float gs = 0.0f, graw = 0.0f;
        bool flp = false;
    };
    auto load_slot = [&](int t, int k) -> SlotIn {
        SlotIn in;
        const int64_t slot = (static_cast<int64_t>(b) * T + t) * K + k;
        in.parent = p.parents[slot];
        in.len = p.lengths[slot];
        in.tok = p.tokens[slot];
        in.flp = p.from_logprob[slot] != 0;
        if (p.g_scores) in.gs = p.g_scores[slot];
        if (p.g_raw) in.graw = p.g_raw[slot];
        return in;
    };
    auto walk_slot = [&](int t, int k, const SlotIn& in) {
        const bool last = t == steps_b - 1;
        const int parent = in.parent;
        const bool valid = k < Kb && parent >= 0 && parent < Kb;  // malformed slots carry nothing
        float d = 0.0f;
        if (valid) {
            float drank = 0.0f;
            if (p.g_scores) drank = drank + in.gs;
            if (last && p.g_final) drank = drank + p.g_final[static_cast<int64_t>(b) * K + k];
            const float inv_pen = 1.0f / length_penalty(in.len, p.alpha);
            d = next[k] + drank * inv_pen;
            if (p.g_raw) d = d + in.graw;
            if (last && p.g_final_raw) d = d + p.g_final_raw[static_cast<int64_t>(b) * K + k];
        }
        const bool flows = valid && d != 0.0f;
        draw[k] = flows ? d : 0.0f;
        par[k] = flows ? parent : -1;
        p.draws[(static_cast<int64_t>(b) * T + t) * K + k] =
            (flows && in.flp && in.tok >= 0 && in.tok < V) ? d : 0.0f;
    };
    const bool one_slot = K <= kWalkThreads;
    SlotIn cur;
    if (one_slot && tid < K && steps_b > 0) cur = load_slot(steps_b - 1, tid);
    for (int t = steps_b - 1; t >= 0; --t) {
        if (one_slot) {
            if (tid < K) {
                SlotIn nxt;
                if (t > 0) nxt = load_slot(t - 1, tid);
                walk_slot(t, tid, cur);
                cur = nxt;
            }
        } else {
            for (int k = tid; k < K; k += kWalkThreads) walk_slot(t, k, load_slot(t, k));
        }
        __syncthreads();
        // each parent sums its children's raw-score gradients in slot order;
        // the sums become the next step's incoming gradients (the two
        // buffers alternate, so one barrier separates the phases)
        for (int q = tid; q < K; q += kWalkThreads) {
            float s = 0.0f;
            for (int k = 0; k < K; ++k)
                if (par[k] == q) s = s + draw[k];
            if (p.pool_d) {
                // then the pool entries of the step with this parent
                const int64_t pb = (static_cast<int64_t>(b) * T + t) * p.P;
                for (int j = 0; j < p.P; ++j) {
                    const float dj = p.pool_d[pb + j];
                    if (dj != 0.0f && p.pool_parents[pb + j] == q) s = s + dj;
                }
            }
            prev[q] = s;
        }
        __syncthreads();
        float* const swap = next;
        next = prev;
        prev = swap;
    }
}

// path_walk_kernel for K <= 64: one wavefront per example walks, lane k
// holding slot k and its incoming gradient in registers, and each parent
// sums its children's raw-score gradients by reading the slots' lanes in slot
// order (v_readlane): the same additions in the same order as the workgroup
// walk, with no barrier and no LDS round trip per step. The next step's slot
// is loaded while a step is walked.
__global__ __launch_bounds__(64) void path_walk_wave_kernel(BackwardParams p) {
    const int b = static_cast<int>(blockIdx.x);
    const int k = static_cast<int>(threadIdx.x);
    const int K = p.K, T = p.T, V = p.V;
    const int steps_b = p.steps ? p.steps[b] : T;
    const int Kb = p.beams ? p.beams[b] : K;  // slots past the example's beams carry nothing
    const int64_t base = static_cast<int64_t>(b) * T * K;
    // steps the example did not decode carry no gradient
    for (int64_t i = static_cast<int64_t>(steps_b) * K + k; i < static_cast<int64_t>(T) * K; i += 64)
        p.draws[base + i] = 0.0f;
    struct SlotIn {
        int parent = -1, len = 0, tok = -1;
        float gs = 0.0f, graw = 0.0f;
        bool flp = false;
    };
    auto load_slot = [&](int t) -> SlotIn {
        SlotIn in;
        const int64_t i = base + static_cast<int64_t>(t) * K + k;
        in.parent = p.parents[i];
        in.len = p.lengths[i];
        in.tok = p.tokens[i];
        in.flp = p.from_logprob[i] != 0;
        if (p.g_scores) in.gs = p.g_scores[i];
        if (p.g_raw) in.graw = p.g_raw[i];
        return in;
    };
    float next = 0.0f;  // the slot's incoming gradient from the later steps
    SlotIn cur;
    if (k < K && steps_b > 0) cur = load_slot(steps_b - 1);
    for (int t = steps_b - 1; t >= 0; --t) {
        SlotIn nxt;
        if (k < K && t > 0) nxt = load_slot(t - 1);
        const bool last = t == steps_b - 1;
        const bool valid = k < K && k < Kb && cur.parent >= 0 && cur.parent < Kb;  // malformed slots carry nothing
        float d = 0.0f;
        if (valid) {
            float drank = 0.0f;
            if (p.g_scores) drank = drank + cur.gs;
            if (last && p.g_final) drank = drank + p.g_final[static_cast<int64_t>(b) * K + k];
            const float inv_pen = 1.0f / length_penalty(cur.len, p.alpha);
            d = next + drank * inv_pen;
            if (p.g_raw) d = d + cur.graw;
            if (last && p.g_final_raw) d = d + p.g_final_raw[static_cast<int64_t>(b) * K + k];
        }
        const bool flows = valid && d != 0.0f;
        const float draw = flows ? d : 0.0f;
        const int par = flows ? cur.parent : -1;
        if (k < K)
            p.draws[base + static_cast<int64_t>(t) * K + k] =
                (flows && cur.flp && cur.tok >= 0 && cur.tok < V) ? d : 0.0f;
        // each parent sums its children's draws in slot order
        float sum = 0.0f;
        for (int j = 0; j < K; ++j) {
            const int pj = __builtin_amdgcn_readlane(par, j);
            const float dj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, draw), j));
            if (pj == k) sum = sum + dj;
        }
        next = sum;
        cur = nxt;
    }
}

// path_walk_wave_kernel with the example's trace in LDS (T * K up to
// kWalkStageSlots). The workgroup's four wavefronts first stage, per slot,
// everything of the walk that does not depend on the later steps, with all
// loads in flight at once: the parent (-1 for a malformed slot), the product
// of the slot's score gradient (the final one added at the last step) and
// its inverse length penalty, the raw-score gradient and whether the draw is
// emitted (from a log-prob entry with a token in range). Wavefront 0 then
// walks reading only LDS, the next step's slot read while a step is walked,
// and writes the draws to LDS; after a barrier the four wavefronts store
// them. The serial loop holds no global memory round trip and no division;
// every value is rounded as in the one-wavefront walk.
constexpr int kWalkStageThreads = 256;
constexpr int kWalkStageSlots = 3072;  // at most 17 bytes a slot in LDS

size_t walk_stage_bytes(const BackwardParams& p) {
    const size_t per = 3 * sizeof(float) + (p.g_raw ? sizeof(float) : 0) + 1;
    return per * static_cast<size_t>(p.T) * static_cast<size_t>(p.K);
}

// KMAX (a power of two >= K): the children loop is unrolled over KMAX lanes;
// lanes from K on hold parent -1, so they match no slot.
template <int KMAX>
__global__ __launch_bounds__(kWalkStageThreads) void path_walk_staged_kernel(BackwardParams p) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float s_gfr[64];
    const int b = static_cast<int>(blockIdx.x);
    const int tid = static_cast<int>(threadIdx.x);
    const int K = p.K, T = p.T, V = p.V;
    const int steps_b = p.steps ? p.steps[b] : T;
    const int Kb = p.beams ? p.beams[b] : K;  // slots past the example's beams carry nothing
    const int64_t base = static_cast<int64_t>(b) * T * K;
    // steps the example did not decode carry no gradient
    for (int64_t i = static_cast<int64_t>(steps_b) * K + tid; i < static_cast<int64_t>(T) * K;
         i += kWalkStageThreads)
        p.draws[base + i] = 0.0f;
    const int n = steps_b * K;
    int32_t* s_par = reinterpret_cast<int32_t*>(smem);
    float* s_a = reinterpret_cast<float*>(s_par + n);
    float* s_draw = s_a + n;
    float* s_graw = s_draw + n;
    uint8_t* s_emit = reinterpret_cast<uint8_t*>(s_graw + (p.g_raw ? n : 0));
    for (int i = tid; i < n; i += kWalkStageThreads) {
        const int64_t g = base + i;
        const int k = i % K;
        const int parent = p.parents[g];
        s_par[i] = k < Kb && parent >= 0 && parent < Kb ? parent : -1;  // malformed slots carry nothing
        float drank = 0.0f;
        if (p.g_scores) drank = drank + p.g_scores[g];
        if (i >= n - K && p.g_final) drank = drank + p.g_final[static_cast<int64_t>(b) * K + k];
        const float inv_pen = 1.0f / length_penalty(p.lengths[g], p.alpha);
        s_a[i] = drank * inv_pen;
        const int tok = p.tokens[g];
        s_emit[i] = p.from_logprob[g] != 0 && tok >= 0 && tok < V;
        if (p.g_raw) s_graw[i] = p.g_raw[g];
    }
    if (tid < K) s_gfr[tid] = p.g_final_raw ? p.g_final_raw[static_cast<int64_t>(b) * K + tid] : 0.0f;
    __syncthreads();
    if (tid < 64) {
        const int k = tid;
        const int kc = k < K ? k : K - 1;  // lanes past K read slot K - 1 and drop it
        struct Slot {
            int par;
            float a, graw;
            bool emit;
        };
        auto read_slot = [&](int t) -> Slot {
            const int i = t * K + kc;
            Slot s;
            s.par = k < K ? s_par[i] : -1;
            s.a = s_a[i];
            s.graw = p.g_raw ? s_graw[i] : 0.0f;
            s.emit = s_emit[i] != 0;
            return s;
        };
        float next = 0.0f;  // the slot's incoming gradient from the later steps
        Slot cur = steps_b > 0 ? read_slot(steps_b - 1) : Slot{-1, 0.0f, 0.0f, false};
        for (int t = steps_b - 1; t >= 0; --t) {
            const Slot nxt = t > 0 ? read_slot(t - 1) : cur;
            float d = 0.0f;
            if (cur.par >= 0) {
                d = next + cur.a;
                if (p.g_raw) d = d + cur.graw;
                if (t == steps_b - 1 && p.g_final_raw) d = d + s_gfr[k];
            }
            const bool flows = cur.par >= 0 && d != 0.0f;
            const float draw = flows ? d : 0.0f;
            const int par = flows ? cur.par : -1;
            if (k < K) s_draw[t * K + k] = (flows && cur.emit) ? d : 0.0f;
            // each parent sums its children's draws in slot order (a child's
            // draw is never +-0, and a sum of them never -0, so adding +0
            // for the other lanes changes nothing)
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j < KMAX; ++j) {
                const int pj = __builtin_amdgcn_readlane(par, j);
                const float dj =
                    __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, draw), j));
                sum = sum + (pj == k ? dj : 0.0f);
            }
            next = sum;
            cur = nxt;
        }
    }
    __syncthreads();
    for (int i = tid; i < n; i += kWalkStageThreads) p.draws[base + i] = s_draw[i];
}

template <int DT>
__device__ __forceinline__ float load_logit(const void* base, int64_t i) {
    if constexpr (DT == 0) {
        return static_cast<const float*>(base)[i];
    } else if constexpr (DT == 1) {
        return half_to_f32(static_cast<const uint16_t*>(base)[i]);
    } else {
        return bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
    }
}

template <int OT>
__device__ __forceinline__ void store_out(void* out, int64_t i, float v, bool accumulate) {
    if constexpr (OT == 0) {
        float* o = static_cast<float*>(out);
        o[i] = accumulate ? o[i] + v : 0.0f + v;
    } else if constexpr (OT == 1) {
        static_cast<uint16_t*>(out)[i] = f32_to_f16_rne(0.0f + v);
    } else {
        static_cast<uint16_t*>(out)[i] = f32_to_bf16_rne(0.0f + v);
    }
}

// Stores zeros over [0, V) of a row (fresh mode): 16-byte stores when the row
// is 16-byte aligned and whole 16-byte blocks long.
template <int OT>
__device__ __forceinline__ void zero_row(void* out, int64_t row_off, int V) {
    const int tid = static_cast<int>(threadIdx.x);
    constexpr int per16 = OT == 0 ? 4 : 8;
    char* row = static_cast<char*>(out) + row_off * (OT == 0 ? 4 : 2);
    if (V % per16 == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0) {
        uint4* r4 = reinterpret_cast<uint4*>(row);
        for (int c = tid; c < V / per16; c += kDenseThreads) r4[c] = make_uint4(0u, 0u, 0u, 0u);
        return;
    }
    for (int v = tid; v < V; v += kDenseThreads) {
        if constexpr (OT == 0) {
            static_cast<float*>(out)[row_off + v] = 0.0f;
        } else {
            static_cast<uint16_t*>(out)[row_off + v] = 0;
        }
    }
}

// POOL: the relaxed pool's entries join the row's (after the selected
// slots' entries of the same token: slot K + j), up to K + P entries a row.
// SMALL: rows of at most 64 entries (K <= 64 without the pool: one entry a
// selected slot at most), whose entry arrays take 768 bytes of LDS instead of
// 12 KB: with the bfloat16 term table (32 KB) four workgroups fit a CU
// instead of three.
template <int DT, int OT, bool LOGITS, bool POOL = false, bool SMALL = false>
__global__ __launch_bounds__(kDenseThreads) void dense_gradient_kernel(BackwardParams p) {
    constexpr int kEntries = SMALL ? 64 : (POOL ? 2 * DBS_CUDA_MAX_BEAM : DBS_CUDA_MAX_BEAM);
    __shared__ int32_t e_tok[kEntries];
    __shared__ float e_val[kEntries];
    __shared__ int32_t e_slot[kEntries];
    __shared__ int n_raw;
    __shared__ int n_ent;
    __shared__ float s_sum;
    const int tid = static_cast<int>(threadIdx.x);
    const int K = p.K, T = p.T, V = p.V;
    // Row (b, t, q). Workgroups go to the eight XCDs in turn (workgroup i to
    // XCD i % 8), and the rows that read their logits are the path rows,
    // which gather on a few parent slots q: with K = 8 they would all land on
    // a few XCDs. Within each group of eight workgroups the rows are rotated
    // by the group's index, which spreads every q over the XCDs.
    const int64_t wg = blockIdx.x;
    const int64_t r = (wg | 7) < static_cast<int64_t>(gridDim.x) ? ((wg & ~int64_t{7}) | ((wg + (wg >> 3)) & 7)) : wg;
    const int b = static_cast<int>(r / (static_cast<int64_t>(T) * K));
    const int t = static_cast<int>((r / K) % T);
    const int q = static_cast<int>(r % K);
    const int steps_b = p.steps ? p.steps[b] : T;
    const int64_t row_off = r * V;
    // p.accumulate: 0 writes every row fresh, 1 adds into float32, 2 writes
    // fresh only the rows that receive an entry (the caller's buffer already
    // holds zeros everywhere else)
    const bool accumulate = p.accumulate == 1;
    const bool zeroed = p.accumulate == 2;

    if (tid == 0) n_raw = 0;
    __syncthreads();
    if (t < steps_b) {
        const int64_t base = (static_cast<int64_t>(b) * T + t) * K;
        for (int k = tid; k < K; k += kDenseThreads) {
            const float d = p.draws[base + k];
            if (d != 0.0f && p.parents[base + k] == q) {
                const int i = atomicAdd(&n_raw, 1);
                e_tok[i] = p.tokens[base + k];
                e_val[i] = d;
                e_slot[i] = k;
            }
        }
        if constexpr (POOL) {
            const int64_t pb = (static_cast<int64_t>(b) * T + t) * p.P;
            for (int j = tid; j < p.P; j += kDenseThreads) {
                const float d = p.pool_d[pb + j];
                const int32_t tok = p.pool_tokens[pb + j];
                if (d != 0.0f && p.pool_parents[pb + j] == q && p.pool_flp[pb + j] && tok >= 0 && tok < V) {
                    const int i = atomicAdd(&n_raw, 1);
                    e_tok[i] = tok;
                    e_val[i] = d;
                    e_slot[i] = K + j;
                }
            }
        }
    }
    __syncthreads();
    if (tid == 0) {
        // order by (token, slot), merge equal tokens in slot order from 0, and
        // sum the row's entries in token order (reference src/decoder.cpp:668-683)
        const int n = n_raw;
        for (int i = 1; i < n; ++i) {
            const int32_t tk = e_tok[i], sl = e_slot[i];
            const float vl = e_val[i];
            int j = i - 1;
            while (j >= 0 && (e_tok[j] > tk || (e_tok[j] == tk && e_slot[j] > sl))) {
                e_tok[j + 1] = e_tok[j];
                e_val[j + 1] = e_val[j];
                e_slot[j + 1] = e_slot[j];
                --j;
            }
            e_tok[j + 1] = tk;
            e_val[j + 1] = vl;
            e_slot[j + 1] = sl;
        }
        int w = 0;
        float total = 0.0f;
        for (int i = 0; i < n;) {
            float v = 0.0f;
            int j = i;
            for (; j < n && e_tok[j] == e_tok[i]; ++j) v = v + e_val[j];
            e_tok[w] = e_tok[i];
            e_val[w] = v;
            ++w;
            total = total + v;
            i = j;
        }
        n_ent = w;
        s_sum = total;
    }
    __syncthreads();
    const int ne = n_ent;

    if (!LOGITS || ne == 0) {
        if (!accumulate && !zeroed) zero_row<OT>(p.out, row_off, V);
        if (ne > 0) {
            __syncthreads();  // the entries land after the zeros of this workgroup
            for (int i = tid; i < ne; i += kDenseThreads) store_out<OT>(p.out, row_off + e_tok[i], e_val[i], accumulate);
        }
        return;
    }

    // From logits: g_v - softmax(x_v) * S over the whole row.
    const float S = s_sum;
    const float lse = p.row_lse[r];
    const size_t esz = DT == 0 ? 4 : 2;
    const void* x = static_cast<const char*>(p.logits) + static_cast<size_t>(r) * static_cast<size_t>(V) * esz;
    if constexpr (DT == 2 && OT != 0) {
        // bfloat16 logits into a 16-bit gradient: exp(fl(x - lse)) is a
        // function of x's pattern for the row, so a per-row table of the exact
        // terms (as in the row pass; table_fits) replaces the Cephes
        // evaluation, and 16-byte loads and stores carry 8 entries. The
        // entries' tokens are written after the rest of the row.
        int ulo = 0;
        const bool vec = (V & 7) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                         (reinterpret_cast<uintptr_t>(p.out) & 15) == 0;
        if (vec && !accumulate && table_fits(lse, ulo)) {
            __shared__ float lut[2 * kLutHalf];
            const uint32_t mp = f32_bits(lse) >> 16;  // largest bfloat16 <= lse (no x exceeds it)
            for (int i = tid; i < 2 * kLutHalf; i += kDenseThreads) {
                const bool neg = i >= kLutHalf;
                const int k = i & (kLutHalf - 1);
                float term = 0.0f;
                if (k == 0) {
                    term = exp_nonpositive(-lse);
                } else {
                    const int u = ulo - 1 + k;
                    if (u < 0x7f80 && (neg || u <= static_cast<int>(mp)))
                        term = exp_nonpositive(bf16_to_f32(static_cast<uint16_t>((neg ? 0x8000 : 0) | u)) - lse);
                }
                lut[i] = term;
            }
            __syncthreads();
            const uint32_t base2 = static_cast<uint32_t>(ulo - 1) * 0x10001u;
            auto terms = [&](uint32_t R, float& lo, float& hi) {
                uint32_t idx = pk_sub_sat_u16(R & 0x7fff7fffu, base2);
                idx = pk_min_u16(idx, 0x0fff0fffu);
                idx |= (R >> 3) & 0x10001000u;
                lo = lut[idx & 0xffffu];
                hi = lut[idx >> 16];
            };
            const uint4* x4 = static_cast<const uint4*>(x);
            uint4* o4 = reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.out) + row_off);
            auto out16 = [&](float g) -> uint32_t {
                return OT == 1 ? f32_to_f16_rne(0.0f + g) : f32_to_bf16_rne(0.0f + g);
            };
            // kDenseBatch 16-byte loads per thread are issued before any store of
            // the batch: the stores may alias the logits as far as the compiler
            // knows, so a load-convert-store loop would wait out one memory
            // latency per block.
            // Two batches alternate: the next batch's loads are in flight while
            // the current one is converted and stored. Every load and store is
            // unconditional, so the compiler's wait counts stay exact (a store
            // under a branch makes it wait for every store before each use of
            // a load): a block index past the row reads and writes the row's
            // last block instead, the same bytes its own thread stores.
            const int n4 = V / 8;
            constexpr int kStride = kDenseBatch * kDenseThreads;
            auto block = [&](int c) __attribute__((always_inline)) { return c < n4 ? c : n4 - 1; };
            auto load_batch = [&](uint4 (&q)[kDenseBatch], int c0) __attribute__((always_inline)) {
#pragma unroll
                for (int u = 0; u < kDenseBatch; ++u) q[u] = x4[block(c0 + u * kDenseThreads)];
            };
            auto store_batch = [&](const uint4 (&q)[kDenseBatch], int c0) __attribute__((always_inline)) {
#pragma unroll
                for (int u = 0; u < kDenseBatch; ++u) {
                    const uint32_t w[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
                    uint32_t o[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float lo, hi;
                        terms(w[e], lo, hi);
                        o[e] = out16(0.0f - lo * S) | (out16(0.0f - hi * S) << 16);
                    }
                    o4[block(c0 + u * kDenseThreads)] = make_uint4(o[0], o[1], o[2], o[3]);
                }
            };
            const int pairs = (n4 + 2 * kStride - 1) / (2 * kStride);
            uint4 qa[kDenseBatch], qb[kDenseBatch];
            load_batch(qa, tid);
            for (int i = 0; i < pairs; ++i) {
                const int ca = tid + 2 * i * kStride;
                load_batch(qb, ca + kStride);
                store_batch(qa, ca);
                load_batch(qa, ca + 2 * kStride);
                store_batch(qb, ca + kStride);
            }
            __syncthreads();  // the entries' tokens land after the rest of the row
            for (int i = tid; i < ne; i += kDenseThreads) {
                const int v = e_tok[i];
                float lo, hi;
                terms(static_cast<const uint16_t*>(x)[v], lo, hi);
                static_cast<uint16_t*>(p.out)[row_off + v] = static_cast<uint16_t>(out16(e_val[i] - lo * S));
            }
            return;
        }
    }
    for (int v0 = tid; v0 < V; v0 += kDenseBatch * kDenseThreads) {
      float xs[kDenseBatch];
#pragma unroll
      for (int u = 0; u < kDenseBatch; ++u) {
          const int v = v0 + u * kDenseThreads;
          xs[u] = v < V ? load_logit<DT>(x, v) : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < kDenseBatch; ++u) {
        const int v = v0 + u * kDenseThreads;
        if (v >= V) break;
        const float pv = softmax_probability(xs[u], lse);
        // entry value of token v, by binary search of the sorted entry tokens
        int lo = 0, hi = ne;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (e_tok[mid] < v) lo = mid + 1;
            else hi = mid;
        }
        const float g = (lo < ne && e_tok[lo] == v) ? e_val[lo] : 0.0f;
        store_out<OT>(p.out, row_off + v, g - pv * S, accumulate);
      }
    }
}

template <int OT>
hipError_t launch_dense_ot(const BackwardParams& p, hipStream_t stream) {
    const int64_t rows = static_cast<int64_t>(p.B) * p.T * p.K;
    if (rows > 0x7fffffffLL) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(rows));
    KernelTimer timer(kKindDense, stream);
    if (p.pool_d) {
        if (!p.logits)
            hipLaunchKernelGGL((dense_gradient_kernel<0, OT, false, true>), grid, dim3(kDenseThreads), 0, stream, p);
        else if (p.logits_type == 0)
            hipLaunchKernelGGL((dense_gradient_kernel<0, OT, true, true>), grid, dim3(kDenseThreads), 0, stream, p);
        else if (p.logits_type == 1)
            hipLaunchKernelGGL((dense_gradient_kernel<1, OT, true, true>), grid, dim3(kDenseThreads), 0, stream, p);
        else
            hipLaunchKernelGGL((dense_gradient_kernel<2, OT, true, true>), grid, dim3(kDenseThreads), 0, stream, p);
    } else if (!p.logits) {
        hipLaunchKernelGGL((dense_gradient_kernel<0, OT, false>), grid, dim3(kDenseThreads), 0, stream, p);
    } else if (p.logits_type == 0) {
        hipLaunchKernelGGL((dense_gradient_kernel<0, OT, true>), grid, dim3(kDenseThreads), 0, stream, p);
    } else if (p.logits_type == 1) {
        hipLaunchKernelGGL((dense_gradient_kernel<1, OT, true>), grid, dim3(kDenseThreads), 0, stream, p);
    } else if (p.K <= 64) {
        hipLaunchKernelGGL((dense_gradient_kernel<2, OT, true, false, true>), grid, dim3(kDenseThreads), 0, stream, p);
    } else {
        hipLaunchKernelGGL((dense_gradient_kernel<2, OT, true>), grid, dim3(kDenseThreads), 0, stream, p);
    }
    return hipGetLastError();
}

// I: the index type of tokens, parents and steps (int32, or int64 as torch
// hands the trace to the caller). STAGED: the example's tokens and parents
// are first copied into LDS by the whole workgroup (coalesced), so each
// beam's walk back through the steps reads the LDS instead of waiting on one
// dependent global load per step. With `lengths` ([B, K] final lengths),
// positions at and past each final beam's length are -1 as well.
template <typename I, bool STAGED>
__global__ void backtrack_kernel(const I* tokens, const I* parents, const I* steps, const I* lengths, int T, int K,
                                 int64_t* seq) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int b = static_cast<int>(blockIdx.x);
    const int64_t steps_b = steps ? static_cast<int64_t>(steps[b]) : T;
    const int64_t base = static_cast<int64_t>(b) * T * K;
    int64_t* s_tok = reinterpret_cast<int64_t*>(smem);
    int32_t* s_par = reinterpret_cast<int32_t*>(smem + sizeof(int64_t) * static_cast<size_t>(T) * K);
    if constexpr (STAGED) {
        for (int i = static_cast<int>(threadIdx.x); i < T * K; i += static_cast<int>(blockDim.x)) {
            s_tok[i] = static_cast<int64_t>(tokens[base + i]);
            const int64_t next = static_cast<int64_t>(parents[base + i]);
            s_par[i] = next >= 0 && next < K ? static_cast<int32_t>(next) : -1;
        }
        __syncthreads();
    }
    for (int k = static_cast<int>(threadIdx.x); k < K; k += static_cast<int>(blockDim.x)) {
        int beam = k;
        int64_t* dst = seq + (static_cast<int64_t>(b) * K + k) * T;
        const int64_t keep = lengths ? static_cast<int64_t>(lengths[static_cast<int64_t>(b) * K + k]) : T;
        for (int t = T - 1; t >= 0; --t) {
            if (t >= steps_b || beam < 0) {
                dst[t] = -1;
                continue;
            }
            const int64_t slot = static_cast<int64_t>(t) * K + beam;
            if constexpr (STAGED) {
                dst[t] = t < keep ? s_tok[slot] : -1;
                beam = s_par[slot];
            } else {
                dst[t] = t < keep ? static_cast<int64_t>(tokens[base + slot]) : -1;
                const int64_t next = static_cast<int64_t>(parents[base + slot]);
                beam = next >= 0 && next < K ? static_cast<int>(next) : -1;  // a malformed parent ends the path
            }
        }
    }
}

}  // namespace

size_t backward_workspace_bytes(int B, int T, int K) {
    const size_t n = static_cast<size_t>(B) * T * K * sizeof(float);
    return ((n + 255) / 256) * 256;
}

hipError_t launch_path_walk(const BackwardParams& p, hipStream_t stream) {
    KernelTimer timer(kKindPathWalk, stream);
    if (p.pool_d) {
        // relaxed-pool terms: the workgroup walk (the only one that adds them)
        hipLaunchKernelGGL(path_walk_kernel, dim3(p.B), dim3(kWalkThreads), 0, stream, p);
    } else if (p.K <= 64 && static_cast<int64_t>(p.T) * p.K <= kWalkStageSlots) {
        const dim3 g(p.B), blk(kWalkStageThreads);
        const size_t lds = walk_stage_bytes(p);
        if (p.K <= 8) hipLaunchKernelGGL(path_walk_staged_kernel<8>, g, blk, lds, stream, p);
        else if (p.K <= 16) hipLaunchKernelGGL(path_walk_staged_kernel<16>, g, blk, lds, stream, p);
        else if (p.K <= 32) hipLaunchKernelGGL(path_walk_staged_kernel<32>, g, blk, lds, stream, p);
        else hipLaunchKernelGGL(path_walk_staged_kernel<64>, g, blk, lds, stream, p);
    } else if (p.K <= 64) {
        hipLaunchKernelGGL(path_walk_wave_kernel, dim3(p.B), dim3(64), 0, stream, p);
    } else {
        hipLaunchKernelGGL(path_walk_kernel, dim3(p.B), dim3(kWalkThreads), 0, stream, p);
    }
    return hipGetLastError();
}

hipError_t launch_dense_gradient(const BackwardParams& p, hipStream_t stream) {
    switch (p.out_type) {
        case 0: return launch_dense_ot<0>(p, stream);
        case 1: return launch_dense_ot<1>(p, stream);
        default: return launch_dense_ot<2>(p, stream);
    }
}

template <typename I>
hipError_t launch_backtrack_t(const I* tokens, const I* parents, const I* steps, const I* lengths, int B, int T, int K,
                              int64_t* seq, hipStream_t stream) {
    const int threads = K < 256 ? ((K + 63) / 64) * 64 : 256;
    KernelTimer timer(kKindBacktrack, stream);
    const size_t staged = (sizeof(int64_t) + sizeof(int32_t)) * static_cast<size_t>(T) * static_cast<size_t>(K);
    if (staged <= 48 * 1024) {
        hipLaunchKernelGGL((backtrack_kernel<I, true>), dim3(B), dim3(threads), staged, stream, tokens, parents, steps,
                           lengths, T, K, seq);
    } else {
        hipLaunchKernelGGL((backtrack_kernel<I, false>), dim3(B), dim3(threads), 0, stream, tokens, parents, steps,
                           lengths, T, K, seq);
    }
    return hipGetLastError();
}

hipError_t launch_backtrack(const int32_t* tokens, const int32_t* parents, const int32_t* steps, int B, int T, int K,
                            int64_t* seq, hipStream_t stream) {
    return launch_backtrack_t<int32_t>(tokens, parents, steps, nullptr, B, T, K, seq, stream);
}

hipError_t launch_backtrack(const int64_t* tokens, const int64_t* parents, const int64_t* steps,
                            const int64_t* lengths, int B, int T, int K, int64_t* seq, hipStream_t stream) {
    return launch_backtrack_t<int64_t>(tokens, parents, steps, lengths, B, T, K, seq, stream);
}

namespace {

constexpr int kRiskThreads = 256;

// The expected cost of one example's beams under softmax(score / t) over its
// live beams (finite scores), and each beam's gradient factor
// scale * p_k (c_k - risk) / t (0 for dead beams). One workgroup per example,
// beams strided over its threads; max and sums by wave reduction, then over
// the wavefronts in LDS.
__global__ __launch_bounds__(kRiskThreads) void risk_kernel(const float* scores, const float* costs, int K,
                                                           float temperature, float scale, float* risk,
                                                           float* factor) {
    __shared__ float s_red[kRiskThreads / 64];
    const int b = static_cast<int>(blockIdx.x);
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63, wave = tid >> 6;
    const float* s = scores + static_cast<int64_t>(b) * K;
    const float* c = costs + static_cast<int64_t>(b) * K;
    auto block_reduce = [&](float v, bool is_max) {
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(v, off);
            v = is_max ? fmaxf(v, o) : v + o;
        }
        if (lane == 0) s_red[wave] = v;
        __syncthreads();
        float r = s_red[0];
        for (int w = 1; w < kRiskThreads / 64; ++w) r = is_max ? fmaxf(r, s_red[w]) : r + s_red[w];
        __syncthreads();
        return r;
    };
    float m = -kInf;
    for (int k = tid; k < K; k += kRiskThreads)
        if (__builtin_fabsf(s[k]) < kInf) m = fmaxf(m, s[k] / temperature);
    m = block_reduce(m, true);
    const float shift = m > -kInf ? m : 0.0f;
    float w_sum = 0.0f;
    for (int k = tid; k < K; k += kRiskThreads)
        if (__builtin_fabsf(s[k]) < kInf) w_sum += expf(s[k] / temperature - shift);
    w_sum = block_reduce(w_sum, false);
    const float inv = w_sum > 0.0f ? 1.0f / w_sum : 0.0f;
    float r = 0.0f;
    for (int k = tid; k < K; k += kRiskThreads)
        if (__builtin_fabsf(s[k]) < kInf) r += expf(s[k] / temperature - shift) * inv * c[k];
    r = block_reduce(r, false);
    for (int k = tid; k < K; k += kRiskThreads) {
        const bool live = __builtin_fabsf(s[k]) < kInf;
        const float p = live ? expf(s[k] / temperature - shift) * inv : 0.0f;
        factor[static_cast<int64_t>(b) * K + k] = live ? scale * p * (c[k] - r) / temperature : 0.0f;
    }
    if (tid == 0) risk[b] = r;
}

// The same for every example of a small batch (K <= 64) in one workgroup,
// then their mean or sum in index order: lane k of a wavefront holds beam k
// (the same lanes, reductions and operations as risk_kernel, so the same
// bits), each wavefront takes every fourth example.
constexpr int kRiskAllMax = 1024;

__global__ __launch_bounds__(kRiskThreads) void risk_all_kernel(const float* scores, const float* costs, int B, int K,
                                                               float temperature, float scale, int reduction,
                                                               float* risk, float* loss, float* factor) {
    __shared__ float s_risk[kRiskAllMax];
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63, wave = tid >> 6;
    // a wavefront's value as risk_kernel's block_reduce gives it: the wave
    // tree, then the other (empty) wavefronts' identities added in order
    auto wave_reduce = [&](float v, bool is_max) {
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(v, off);
            v = is_max ? fmaxf(v, o) : v + o;
        }
        for (int w = 1; w < kRiskThreads / 64; ++w) v = is_max ? fmaxf(v, -kInf) : v + 0.0f;
        return v;
    };
    for (int b = wave; b < B; b += kRiskThreads / 64) {
        const bool in = lane < K;
        const float sv = in ? scores[static_cast<int64_t>(b) * K + lane] : 0.0f;
        const float cv = in ? costs[static_cast<int64_t>(b) * K + lane] : 0.0f;
        const bool live = in && __builtin_fabsf(sv) < kInf;
        const float m = wave_reduce(live ? sv / temperature : -kInf, true);
        const float shift = m > -kInf ? m : 0.0f;
        const float w_sum = wave_reduce(live ? expf(sv / temperature - shift) : 0.0f, false);
        const float inv = w_sum > 0.0f ? 1.0f / w_sum : 0.0f;
        const float r = wave_reduce(live ? expf(sv / temperature - shift) * inv * cv : 0.0f, false);
        if (in) {
            const float pk = live ? expf(sv / temperature - shift) * inv : 0.0f;
            factor[static_cast<int64_t>(b) * K + lane] = live ? scale * pk * (cv - r) / temperature : 0.0f;
        }
        if (lane == 0) {
            s_risk[b] = r;
            risk[b] = r;
        }
    }
    __syncthreads();
    if (tid == 0 && loss) {
        float acc = 0.0f;
        for (int b = 0; b < B; ++b) acc = acc + s_risk[b];
        loss[0] = reduction == 1 ? acc / static_cast<float>(B) : acc;
    }
}

// Mean (reduction 1) or sum of risk[0, B): each thread sums a contiguous
// slice in order, then the slices are added in order (one workgroup).
__global__ __launch_bounds__(kRiskThreads) void risk_sum_kernel(const float* risk, int B, int reduction, float* loss) {
    __shared__ float s_part[kRiskThreads];
    const int tid = static_cast<int>(threadIdx.x);
    const int per = (B + kRiskThreads - 1) / kRiskThreads;
    float acc = 0.0f;
    for (int i = tid * per; i < B && i < (tid + 1) * per; ++i) acc = acc + risk[i];
    s_part[tid] = acc;
    __syncthreads();
    if (tid == 0) {
        float total = 0.0f;
        for (int i = 0; i < kRiskThreads; ++i) total = total + s_part[i];
        loss[0] = reduction == 1 ? total / static_cast<float>(B) : total;
    }
}

}  // namespace

hipError_t launch_risk(const float* scores, const float* costs, int B, int K, float temperature, int reduction,
                       float* risk, float* loss, float* factor, hipStream_t stream) {
    const float scale = reduction == 1 ? 1.0f / static_cast<float>(B) : 1.0f;
    if (B <= kRiskAllMax && K <= 64) {
        hipLaunchKernelGGL(risk_all_kernel, dim3(1), dim3(kRiskThreads), 0, stream, scores, costs, B, K, temperature,
                           scale, reduction, risk, reduction != 0 ? loss : nullptr, factor);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(risk_kernel, dim3(B), dim3(kRiskThreads), 0, stream, scores, costs, K, temperature, scale,
                       risk, factor);
    if (reduction != 0 && loss) hipLaunchKernelGGL(risk_sum_kernel, dim3(1), dim3(kRiskThreads), 0, stream, risk, B,
                                                   reduction, loss);
    return hipGetLastError();
}

}  // namespace dbs_hip
