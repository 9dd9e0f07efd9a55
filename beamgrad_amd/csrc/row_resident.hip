// SPDX-License-Identifier: MIT
//
// Row pass for 16-bit rows that reads every row from HBM once.
//
// The logsumexp of the reference folds exp(x - max) into 256 lanes (lane j =
// v mod 256, increasing v; reference src/kernels_scalar.cpp:48-66), so the
// row maximum is needed before the first term and each lane's sum is one
// sequential chain. The two-pass kernel (row_pass.hip) streams the row twice;
// on MI355X the second read is not served from cache, which halves the
// attainable rate. Here one 512-thread workgroup per CU keeps a whole row in
// VGPRs while it works on it, persistent over rows:
//
//   * thread (seg, j) owns lane j of the stripes [seg*P, seg*P + P) of the row
//     (stripe s = elements 256 s .. 256 s + 255), packed two stripes per VGPR;
//   * each wavefront streams its 64 lanes in chunks of 8 stripes: one 16-byte
//     global->LDS load per lane moves a chunk (1 KB) into a ring of LDS slots,
//     kRing chunks in flight per wavefront, and the lanes read their own
//     elements back transposed;
//   * packed 16-bit integer max/min over the raw patterns give the row
//     maximum, the NaN/+inf flag and per-register-group maxima;
//   * from logits (bfloat16), exp(fl(x - max)) is a function of x's 16-bit
//     pattern for the row: a per-row table of the exact terms replaces the
//     Cephes evaluation, and the two segments fold their lanes in order
//     (segment 0, then segment 1 continuing the same accumulators);
//   * one wavefront finishes the row: the fixed lane tree, the shortlist.
//
// The table: with E the exponent of the maximum m (m >= 1), every |x| <
// 2^(E-25) gives fl(x - m) = -m, so magnitudes are indexed from u_lo, the
// bfloat16 pattern of 2^(E-25): slot 0 holds exp(-m), slot k >= 1 magnitude
// u_lo - 1 + k; 4096 slots per sign. Positive x never exceeds m (at most 25
// binades above u_lo); negative slots past the last must give 0 (checked per
// row), so magnitudes beyond the table clamp to a zero slot. Rows where this
// does not hold fold with the Cephes evaluation instead.
#include <hip/hip_runtime.h>

#include "device_common.hpp"

namespace dbs_hip {

namespace {

constexpr int kResThreads = 512;                 // two segments of the 256 lanes
constexpr int kResRegs = 152;                    // packed element pairs per thread
constexpr int kResChunks = kResRegs / 4;         // 8-stripe chunks per thread
constexpr int kResGroups = 4;                    // register groups with their own maxima
constexpr int kResGroupRegs = kResRegs / kResGroups;
constexpr int kRing = 8;                         // 1 KB staging slots per wavefront
constexpr int kLutHalf = 4096;                   // table slots per sign
constexpr int kMaxStripes = 2 * 8 * kResChunks;  // 608 stripes: V <= 155648

// LDS layout (bytes). The table sits at 0 so its reads use the immediate offset.
constexpr int kOffLut = 0;
constexpr int kOffRing = kOffLut + 2 * kLutHalf * 4;
constexpr int kOffLaneMax = kOffRing + 8 * kRing * 1024;
constexpr int kOffAcc = kOffLaneMax + 2 * 256 * 4;
constexpr int kOffKey = kOffAcc + 256 * 4;
constexpr int kOffX = kOffKey + kSurvivorCap * 8;
constexpr int kOffWave = kOffX + kSurvivorCap * 4;
constexpr int kOffMisc = kOffWave + 8 * 8;
constexpr int kResLds = kOffMisc + 16;

typedef short v2i16 __attribute__((ext_vector_type(2)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_max_i16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(v2i16, a), __builtin_bit_cast(v2i16, b)));
}
__device__ __forceinline__ uint32_t pk_min_i16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(v2i16, a), __builtin_bit_cast(v2i16, b)));
}
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(v2u16, a), __builtin_bit_cast(v2u16, b)));
}
__device__ __forceinline__ uint32_t pk_min_u16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(v2u16, a), __builtin_bit_cast(v2u16, b)));
}
__device__ __forceinline__ uint32_t pk_sub_sat_u16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(__builtin_bit_cast(v2u16, a), __builtin_bit_cast(v2u16, b)));
}
__device__ __forceinline__ uint32_t pk_sub_sat_i16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(__builtin_bit_cast(v2i16, a), __builtin_bit_cast(v2i16, b)));
}
__device__ __forceinline__ uint32_t pk_sign_fill_i16(uint32_t a) {
    const v2i16 fifteen = {15, 15};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2i16, a) >> fifteen);
}
__device__ __forceinline__ uint32_t pk_shl2_u16(uint32_t a) {
    const v2u16 two = {2, 2};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2u16, a) << two);
}

// Waits until at most N vector-memory operations of the wavefront are
// outstanding (the global->LDS loads complete in issue order) / until its
// LDS reads have returned. The memory clobber keeps the compiler from moving
// LDS accesses across the wait.
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ void load_chunk_lds(const uint16_t* src, unsigned char* dst) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(dst), 16, 0, 0);
}

template <int DT>
__device__ __forceinline__ float pattern_value(uint32_t h) {
    return DT == 1 ? half_to_f32(static_cast<uint16_t>(h)) : bf16_to_f32(static_cast<uint16_t>(h));
}

// Largest value of a register group from its packed signed maxima and minima:
// per half, the largest non-negative pattern, else (all negative) the
// smallest magnitude, which is the smallest signed pattern.
template <int DT>
__device__ __forceinline__ float group_value(uint32_t gmax, uint32_t gmin) {
    float best = -kInf;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int16_t smax = static_cast<int16_t>(gmax >> (16 * h));
        const int16_t smin = static_cast<int16_t>(gmin >> (16 * h));
        const uint32_t pat = static_cast<uint16_t>(smax >= 0 ? smax : smin);
        best = fmaxf(best, pattern_value<DT>(pat));
    }
    return best;
}

// Signed 16-bit key of a sign-magnitude pattern, monotone in its value (-0
// one below +0).
__device__ __forceinline__ int key16(uint32_t h) {
    const int s = static_cast<int16_t>(h);
    return s < 0 ? (s ^ 0x7fff) : s;
}

// The 16-bit pattern of theta (a value of the row, or -inf).
template <int DT>
__device__ __forceinline__ uint32_t value_pattern(float x) {
    return DT == 2 ? (f32_bits(x) >> 16) : f32_to_f16_rne(x);
}

// Whether the bfloat16 term table covers a row with maximum m; u_lo out.
__device__ __forceinline__ bool table_fits(float m, int& ulo) {
    if (!(m >= 1.0f && m < kInf)) return false;
    const uint32_t mp = f32_bits(m) >> 16;
    const int E = static_cast<int>((mp >> 7) & 0xffu) - 127;
    ulo = (E + 102) << 7;
    const int ucap = ulo - 1 + (kLutHalf - 1);
    if (ucap >= 0x7f80) return true;  // the clamp slot is -inf/NaN: term 0
    const float d = bf16_to_f32(static_cast<uint16_t>(0x8000 | ucap)) - m;
    return !(d >= -87.0f);
}

template <int DT, bool LOGITS>
__global__ __launch_bounds__(kResThreads) void row_resident_kernel(DecodeParams p, int64_t rows) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    float* lut = reinterpret_cast<float*>(lds + kOffLut);
    float* s_lane_max = reinterpret_cast<float*>(lds + kOffLaneMax);
    float* s_acc = reinterpret_cast<float*>(lds + kOffAcc);
    uint64_t* s_key = reinterpret_cast<uint64_t*>(lds + kOffKey);
    float* s_x = reinterpret_cast<float*>(lds + kOffX);
    float* s_wmax = reinterpret_cast<float*>(lds + kOffWave);
    int* s_wbad = reinterpret_cast<int*>(lds + kOffWave + 32);
    int* s_count = reinterpret_cast<int*>(lds + kOffMisc);
    float* s_theta = reinterpret_cast<float*>(lds + kOffMisc + 4);

    const int tid = static_cast<int>(threadIdx.x);
    const int j = tid & 255, l = tid & 63;
    // wavefront-uniform: segment, wavefront, wavefront within the segment
    const int seg = __builtin_amdgcn_readfirstlane(tid >> 8);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wv = wave & 3;
    const int V = p.V, M = p.M;
    const int S = (V + 255) >> 8;
    const int per = ((((S + 1) >> 1) + 7) >> 3) << 3;
    const int s_begin = seg * per;
    const int seg_stripes = max(0, min(S, s_begin + per) - s_begin);
    const int nch = (seg_stripes + 7) >> 3;
    constexpr uint32_t kPad = DT == 2 ? 0xff80u : 0xfc00u;    // -inf
    constexpr int kPosInf = DT == 2 ? 0x7f80 : 0x7c00;
    constexpr uint32_t kNegInf = kPad;
    unsigned char* ring = lds + kOffRing + wave * (kRing * 1024);

    if (tid == 0) *s_count = 0;
    __syncthreads();

    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        int b, new_len;
        if (!row_is_read(p, r, b, new_len)) continue;
        const bool mask_eos = new_len < p.min_length;
        const uint16_t* row = static_cast<const uint16_t*>(p.x) + r * V;
        // Opaque copies per row: everything the unrolled load derives from
        // them is recomputed per row instead of being hoisted out of the row
        // loop into (spilled) registers.
        int nch_r = nch, V_r = V, jr = j, lr = l;
        asm volatile("" : "+s"(nch_r), "+s"(V_r));
        asm volatile("" : "+v"(jr), "+v"(lr));

        // ---- load: ring of 1 KB chunks per wavefront, transposed to lanes ----
        // registers past the segment's chunks hold -inf pairs (term 0, never
        // a survivor), so the chain below runs over all of them unguarded
        uint32_t reg[kResRegs];
#pragma unroll
        for (int k = 0; k < kResRegs; ++k) reg[k] = kPad | (kPad << 16);
        uint32_t gmax[kResGroups], gmin[kResGroups];
        uint32_t umax = 0;
#pragma unroll
        for (int g = 0; g < kResGroups; ++g) {
            gmax[g] = 0x80008000u;
            gmin[g] = kPad | (kPad << 16);
        }
        // lane l of the wavefront moves 8 elements: stripe 8c + l/8 of the
        // segment, lanes 64 wv + 8 (l % 8) ...; a group past the row end
        // reads the row start instead (V % 8 == 0: groups are whole) and is
        // replaced by padding below.
        const int v_lane = 256 * (s_begin + (lr >> 3)) + 64 * wv + 8 * (lr & 7);
        auto chunk_src = [&](int c) -> const uint16_t* {
            const int v = v_lane + 2048 * c;
            return row + (v < V_r ? v : 0);
        };
#pragma unroll
        for (int c = 0; c < kRing; ++c)
            if (c < nch_r) load_chunk_lds(chunk_src(c), ring + c * 1024);
#pragma unroll
        for (int c = 0; c < kResChunks; ++c) {
            if (c < nch_r) {
                if (c + kRing < nch_r) wait_vm<kRing - 1>();
                else wait_vm<0>();
                const unsigned char* slot = ring + (c % kRing) * 1024;
                uint32_t e[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) e[i] = *reinterpret_cast<const uint16_t*>(slot + 128 * i + 2 * lr);
                const int sb = s_begin + 8 * c;
                if (256 * (sb + 8) > V_r) {
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        if (256 * (sb + i) + jr >= V_r) e[i] = kPad;
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int k = 4 * c + q;
                    const uint32_t R = e[2 * q] | (e[2 * q + 1] << 16);
                    reg[k] = R;
                    const int g = k / kResGroupRegs;
                    gmax[g] = pk_max_i16(gmax[g], R);
                    gmin[g] = pk_min_i16(gmin[g], R);
                    umax = pk_max_u16(umax, R);
                }
                wait_lds();
                if (c + kRing < nch_r) load_chunk_lds(chunk_src(c + kRing), ring + (c % kRing) * 1024);
            }
        }

        // ---- row maximum, flag, lane maxima ----
        float gval[kResGroups];
        float tmax = -kInf;
        uint32_t allmax = 0x80008000u;
#pragma unroll
        for (int g = 0; g < kResGroups; ++g) {
            gval[g] = group_value<DT>(gmax[g], gmin[g]);
            tmax = fmaxf(tmax, gval[g]);
            allmax = pk_max_i16(allmax, gmax[g]);
        }
        const bool bad = static_cast<int16_t>(allmax & 0xffffu) >= kPosInf ||
                         static_cast<int16_t>(allmax >> 16) >= kPosInf || (umax & 0xffffu) > kNegInf ||
                         (umax >> 16) > kNegInf;
        s_lane_max[seg * 256 + j] = tmax;
        const float wmax = wave_max(tmax);
        const bool wbad = __any(bad);
        if (l == 0) {
            s_wmax[wave] = wmax;
            s_wbad[wave] = wbad ? 1 : 0;
        }
        __syncthreads();

        float m = -kInf;
        bool any_bad = false;
#pragma unroll
        for (int w = 0; w < kResThreads / 64; ++w) {
            m = fmaxf(m, s_wmax[w]);
            any_bad = any_bad || s_wbad[w] != 0;
        }
        if (any_bad) {
            // NaN or +inf in the row: the maxima are over x < +inf (reference
            // src/kernels_scalar.cpp:48-56), so re-read the segment for them;
            // every group is scanned for survivors.
            float lm = -kInf;
            for (int s = s_begin; s < s_begin + 8 * nch; s += 8) {
                float xs[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int v = 256 * (s + u) + j;
                    xs[u] = v < V ? load_one<DT>(row, v) : -kInf;
                }
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (xs[u] < kInf && xs[u] > lm) lm = xs[u];
            }
            __syncthreads();  // every read of the wavefront maxima above is done
            s_lane_max[seg * 256 + j] = lm;
            const float wm = wave_max(lm);
            if (l == 0) s_wmax[wave] = wm;
            __syncthreads();
            m = -kInf;
#pragma unroll
            for (int w = 0; w < kResThreads / 64; ++w) m = fmaxf(m, s_wmax[w]);
#pragma unroll
            for (int g = 0; g < kResGroups; ++g) gval[g] = kInf;
        }
        if (M > 0 && wave == 0) {
            float a[4];
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) a[e2] = fmaxf(s_lane_max[4 * l + e2], s_lane_max[256 + 4 * l + e2]);
            const float th = shortlist_threshold(a, l, M);
            if (l == 0) *s_theta = th;
        }
        int ulo = 0;
        const bool do_lse = LOGITS && m > -kInf;
        const bool use_table = DT == 2 && do_lse && table_fits(m, ulo);
        if (use_table) {
            const uint32_t mp = f32_bits(m) >> 16;
            for (int s = tid; s < 2 * kLutHalf; s += kResThreads) {
                const bool neg = s >= kLutHalf;
                const int k = s & (kLutHalf - 1);
                float term = 0.0f;
                if (k == 0) {
                    term = exp_nonpositive(-m);
                } else {
                    const int u = ulo - 1 + k;
                    if (u < 0x7f80 && (neg || u <= static_cast<int>(mp)))
                        term = exp_nonpositive(bf16_to_f32(static_cast<uint16_t>((neg ? 0x8000 : 0) | u)) - m);
                }
                lut[s] = term;
            }
        }
        __syncthreads();
        const float theta = M > 0 ? *s_theta : kInf;

        // ---- registers holding x >= theta (groups whose maximum reaches it) ----
        // A packed key test marks them (a superset: keys >= key(theta) - 1, so
        // -0 and +0 both pass); their elements are re-read from the row, which
        // is still in cache, while the other segment folds its lanes.
        uint32_t hm[(kResRegs + 31) / 32] = {};
        if (M > 0) {
            int tk = key16(value_pattern<DT>(theta)) - 1;
            if (tk < -32768) tk = -32768;
            const uint32_t tk2 = static_cast<uint32_t>(static_cast<uint16_t>(tk)) * 0x10001u;
#pragma unroll
            for (int g = 0; g < kResGroups; ++g) {
                if (gval[g] >= theta) {
#pragma unroll
                    for (int q = 0; q < kResGroupRegs; ++q) {
                        const int k = g * kResGroupRegs + q;
                        const uint32_t R = reg[k];
                        const uint32_t key = R ^ (pk_sign_fill_i16(R) & 0x7fff7fffu);
                        const uint32_t d = pk_sub_sat_i16(key, tk2) & 0x80008000u;
                        hm[k >> 5] |= (d != 0x80008000u ? 1u : 0u) << (k & 31);
                    }
                }
            }
        }
        auto push_hits = [&]() {
#pragma unroll
            for (int w = 0; w < (kResRegs + 31) / 32; ++w) {
                uint32_t bits = hm[w];
                while (bits != 0u) {
                    const int k = 32 * w + __builtin_ctz(bits);
                    bits &= bits - 1u;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int v = 256 * (s_begin + 2 * k + h) + j;
                        const float x = v < V ? load_one<DT>(row, v) : -kInf;
                        if (x >= theta && x < kInf && x > -kInf) {
                            // banned / EOS-below-min_length tokens are dropped when the row is finished
                            const int slot = atomicAdd(s_count, 1);
                            if (slot < kSurvivorCap) {
                                s_key[slot] = survivor_key(x, v);
                                s_x[slot] = x;
                            }
                        }
                    }
                }
            }
        };

        // ---- the lane chains: segment 0, then segment 1 ----
        // Segment 1 records its survivors, then waits at its first barrier
        // until segment 0 has folded its stripes; each wavefront passes the
        // same two barriers.
        if (seg == 1) {
            push_hits();
            __syncthreads();
        }
        if (do_lse) {
            float acc = seg == 0 ? 0.0f : s_acc[j];
            if (use_table) {
                // table index of a pattern: magnitude - (u_lo - 1) saturated at
                // 0 (slot 0) and clamped to 4095, plus 4096 for negative x; the
                // two halves of a register at once
                const uint32_t base2 = static_cast<uint32_t>(ulo - 1) * 0x10001u;
                auto lookup = [&](int k, float& lo, float& hi) {
                    const uint32_t R = reg[k];
                    uint32_t idx = pk_sub_sat_u16(R & 0x7fff7fffu, base2);
                    idx = pk_min_u16(idx, 0x0fff0fffu);
                    idx |= (R >> 3) & 0x10001000u;
                    const uint32_t addr = pk_shl2_u16(idx);
                    lo = *reinterpret_cast<const float*>(lds + kOffLut + (addr & 0xffffu));
                    hi = *reinterpret_cast<const float*>(lds + kOffLut + (addr >> 16));
                };
                // blocks of kBlk registers; the lookups of block b + 1 are in
                // flight while block b is added in order
                constexpr int kBlk = 4;
                float cur[2 * kBlk], nxt[2 * kBlk];
#pragma unroll
                for (int q = 0; q < kBlk; ++q) lookup(q, cur[2 * q], cur[2 * q + 1]);
#pragma unroll
                for (int k0 = 0; k0 < kResRegs; k0 += kBlk) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (k0 + kBlk < kResRegs) {
#pragma unroll
                        for (int q = 0; q < kBlk; ++q) lookup(k0 + kBlk + q, nxt[2 * q], nxt[2 * q + 1]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int q = 0; q < 2 * kBlk; ++q) acc = acc + cur[q];
#pragma unroll
                    for (int q = 0; q < 2 * kBlk; ++q) cur[q] = nxt[q];
                }
            } else {
                // Cephes terms, re-reading the segment (its lines are still cached)
                for (int s = s_begin; s < s_begin + 8 * nch; s += 8) {
                    float xs[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int v = 256 * (s + u) + j;
                        xs[u] = v < V ? load_one<DT>(row, v) : -kInf;
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        if (xs[u] < kInf && xs[u] > -kInf) acc = acc + exp_nonpositive(xs[u] - m);
                }
            }
            s_acc[j] = acc;
        }
        if (seg == 0) {
            __syncthreads();
            push_hits();
        }
        __syncthreads();

        // ---- finish: lane tree, shortlist, RowInfo ----
        if (wave == 0) {
            float lse = 0.0f;
            if (LOGITS) {
                if (do_lse) {
                    float a[4];
#pragma unroll
                    for (int e2 = 0; e2 < 4; ++e2) a[e2] = s_acc[4 * l + e2];
                    lse = logsumexp_from(m, lane_tree_sum(a, l));
                } else {
                    lse = -kInf;
                }
            }
            const int n = *s_count;
            finish_row_wave<LOGITS, true>(p, r, lse, theta, any_bad, s_key, s_x, n, l, b, mask_eos);
            wave_sync();
            if (l == 0) *s_count = 0;
        }
    }
}

int g_cu_count[64];

template <int DT, bool LOGITS>
hipError_t launch_resident(const DecodeParams& p, int64_t rows, int device, hipStream_t stream) {
    static bool attr_set[64] = {};
    if (!attr_set[device]) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&row_resident_kernel<DT, LOGITS>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, kResLds);
        if (e != hipSuccess) return e;
        attr_set[device] = true;
    }
    const int64_t grid = rows < g_cu_count[device] ? rows : g_cu_count[device];
    hipLaunchKernelGGL((row_resident_kernel<DT, LOGITS>), dim3(static_cast<unsigned>(grid)), dim3(kResThreads),
                       kResLds, stream, p, rows);
    return hipGetLastError();
}

}  // namespace

bool row_resident_eligible(const DecodeParams& p) {
    if (p.dtype != 1 && p.dtype != 2) return false;
    if (p.V % 8 != 0 || reinterpret_cast<uintptr_t>(p.x) % 16 != 0) return false;
    if ((p.V + 255) / 256 > kMaxStripes) return false;
    return p.M <= 256;
}

hipError_t launch_row_resident(const DecodeParams& p, int64_t rows, hipStream_t stream) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    if (g_cu_count[device] == 0) {
        int cus = 0;
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
        if (e != hipSuccess) return e;
        g_cu_count[device] = cus > 0 ? cus : 1;
    }
    if (p.from_logits) return p.dtype == 2 ? launch_resident<2, true>(p, rows, device, stream)
                                           : launch_resident<1, true>(p, rows, device, stream);
    return p.dtype == 2 ? launch_resident<2, false>(p, rows, device, stream)
                        : launch_resident<1, false>(p, rows, device, stream);
}

}  // namespace dbs_hip
