// SPDX-License-Identifier: MIT
//
// Pipelined row pass for 16-bit rows: every row is read from HBM once, and
// the next rows stream in while the current one is folded.
//
// The logsumexp of the reference folds exp(x - max) into 256 lanes (lane j =
// v mod 256, increasing v; reference src/kernels_scalar.cpp:48-66): the row
// maximum is needed before the first term, and each lane's sum is one
// sequential chain. One 512-thread workgroup per CU, persistent over rows,
// keeps the row it works on in VGPRs:
//
//   * the row is cut into 512-byte windows (256 positions; position p holds
//     element p - sh, where sh = 1 when the row starts 2 bytes past a 4-byte
//     boundary); the windows form four segments, one per wavefront pair;
//   * thread t of a segment holds the dword at byte 4t of each of its
//     windows: two elements, the lanes 2t - sh and 2t + 1 - sh (mod 256), so
//     one plain coalesced load per window brings them, packed, into the
//     register they are folded from; the thread keeps both lanes' sums;
//   * the segments fold in order (segment g continues the sums of segment
//     g - 1). A segment that has folded its windows loads its windows of the
//     next row into the registers it freed while the later segments fold;
//     segment 0, which folds first, takes the next row from an LDS staging
//     area instead, and refills that area two rows ahead by global->LDS
//     loads, so a row's first quarter is already on chip when the row
//     starts;
//   * packed 16-bit integer max/min over the raw patterns give the row
//     maximum, the NaN/+inf flag and per-register-group maxima; the
//     shortlist threshold theta is the M-th largest of the 512 thread maxima,
//     radix-selected over their 16-bit keys;
//   * from logits (bfloat16), exp(fl(x - max)) is a function of x's 16-bit
//     pattern for the row: a per-row table of the exact terms (see
//     table_fits) replaces the Cephes evaluation; other rows evaluate it;
//   * one wavefront finishes the row: the fixed lane tree, the shortlist.
#include <hip/hip_runtime.h>

#include "row_helpers.hpp"

namespace dbs_hip {

namespace {

constexpr int kPipeThreads = 512;
constexpr int kSegs = 4;                       // window segments, one per wavefront pair
constexpr int kMaxWin = 152;                   // windows per segment (one VGPR each), at most
constexpr int kGroups = 4;                     // register groups with their own maxima
constexpr int kStageDwords = 2 * kMaxWin * 64; // segment 0's windows of a row, per wavefront
constexpr int kBlk = 4;                        // registers whose lookups run ahead of the sums

// The row from its 4-byte aligned start, as seen by one segment.
struct SegView {
    __amdgpu_buffer_rsrc_t rs;  // windows [w_begin, w_begin + P) of the row; reads past them give zeros
    int sh;                     // position p holds element p - sh
};

__device__ __forceinline__ SegView seg_view(const DecodeParams& p, int64_t r, int w_begin, int P) {
    const int64_t e0 = r * static_cast<int64_t>(p.V);
    const int sh = static_cast<int>(e0 & 1);
    const uint16_t* a = static_cast<const uint16_t*>(p.x) + (e0 - sh) + 256 * static_cast<int64_t>(w_begin);
    // bytes of the row from the segment's first window, rounded up to whole
    // 16-byte blocks (a block holding a row byte never crosses a page)
    const int row_bytes = (2 * (p.V + sh) + 15) & ~15;
    const int nbytes = max(0, min(row_bytes - 512 * w_begin, 512 * P));
    return SegView{__builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a), 0, nbytes, 0x00020000), sh};
}

// NW: registers (windows) per segment; every loop over them is unrolled, and
// those past the row's windows hold padding.
template <int DT, bool LOGITS, int NW>
__global__ __launch_bounds__(kPipeThreads) void row_pipe_kernel(DecodeParams p, int64_t rows) {
    static_assert(NW % kGroups == 0 && NW % kBlk == 0 && NW <= kMaxWin, "window layout");
    constexpr int kWin = NW;
    constexpr int kGroupRegs = kWin / kGroups;
    __shared__ __attribute__((aligned(16))) float lut[2 * kLutHalf];
    __shared__ __attribute__((aligned(16))) uint32_t s_stage[kStageDwords];
    // lane sums and survivors by row parity: a row is finished while the
    // next one already folds and records survivors
    __shared__ float s_acc2[2 * 256];
    __shared__ uint64_t s_key2[2 * kSurvivorCap];
    __shared__ float s_x2[2 * kSurvivorCap];
    __shared__ __attribute__((aligned(16))) int s_hist[2 * 256];
    __shared__ int s_wave[16];
    __shared__ int s_count2[2];
    int* s_hist1 = s_hist;
    int* s_hist2 = s_hist + 256;
    int* s_wkey = s_wave;
    int* s_wbad = s_wave + 8;

    const int tid = static_cast<int>(threadIdx.x);
    const int l = tid & 63;
    // wavefront-uniform: segment, wavefront, wavefront within the segment
    const int seg = __builtin_amdgcn_readfirstlane(tid >> 7);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wv = wave & 1;
    const int t = tid & 127;  // positions 2t, 2t + 1 of each window of the segment
    const int V = p.V, M = p.M;
    const int W = (V + 256) >> 8;  // windows of any row (positions < V + 1)
    const int P = (W + kSegs - 1) / kSegs;
    const int w_begin = seg * P;
    const int nwin = max(0, min(W, w_begin + P) - w_begin);  // this segment's windows
    constexpr uint32_t kPad = DT == 2 ? 0xff80u : 0xfc00u;    // -inf
    constexpr uint32_t kPad2 = kPad | (kPad << 16);
    constexpr int kPosInf = DT == 2 ? 0x7f80 : 0x7c00;
    constexpr uint32_t kNegInf = kPad;
    // this wavefront's staging area: dword 64 i + l holds its lanes' dword of window i
    uint32_t* stage = s_stage + wv * (kMaxWin * 64);

    if (tid < 2) s_count2[tid] = 0;
    if (tid < 256) {
        s_hist1[tid] = 0;
        s_hist2[tid] = 0;
    }
    __syncthreads();

    // Wavefront 0 finishes row r (lane tree, shortlist, RowInfo) during the
    // next row, after it has folded its windows of that row and before it
    // takes the row after from the staging area: its registers are free.
    bool pend = false;
    int64_t pend_r = 0;
    float pend_m = 0.0f, pend_theta = 0.0f;
    bool pend_bad = false, pend_lse = false, pend_mask = false, pend_full = false;
    int pend_b = 0, pend_par = 0;
    auto finish_pending = [&]() {
        float lse = 0.0f;
        const float* acc = s_acc2 + 256 * pend_par;
        if (LOGITS) {
            if (pend_lse) {
                float a[4];
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) a[e2] = acc[4 * l + e2];
                lse = logsumexp_from(pend_m, lane_tree_sum(a, l));
            } else {
                lse = -kInf;
            }
        }
        int* cnt = s_count2 + pend_par;
        const int n = pend_full ? kSurvivorCap + 1 : *cnt;
        finish_row_wave<LOGITS, true>(p, pend_r, lse, pend_theta, pend_bad, s_key2 + kSurvivorCap * pend_par,
                                      s_x2 + kSurvivorCap * pend_par, n, l, pend_b, pend_mask);
        wave_sync();
        if (l == 0) *cnt = 0;
        pend = false;
    };

    uint32_t reg[kWin];
    // The segment's windows of row rr, straight into the registers (the
    // compiler waits for each before its first use).
    auto load_windows = [&](int64_t rr) {
        const SegView sv = seg_view(p, rr, w_begin, P);
        int voff = 4 * t;
        asm volatile("" : "+v"(voff));
#pragma unroll
        for (int i = 0; i < kWin; ++i) reg[i] = __builtin_amdgcn_raw_buffer_load_b32(sv.rs, voff, 512 * i, 0);
    };
    // Segment 0's windows of row rr into this wavefront's staging area: each
    // 16-byte load of lane L brings dwords 4 (L % 16) .. + 3 of the
    // wavefront's half of window 4 q + L / 16 (64 lanes = 1 KB = 4 windows).
    auto stage_windows = [&](int64_t rr) {
        const SegView sv = seg_view(p, rr, 0, P);
        int voff = 512 * (l >> 4) + 256 * wv + 16 * (l & 15);
        asm volatile("" : "+v"(voff));
        for (int q = 0; 4 * q < nwin; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                sv.rs, (__attribute__((address_space(3))) void*)(stage + 256 * q), 16, voff, 2048 * q, 0, 0);
    };

    // the row sequence (thread 0 finds it two rows ahead; three slots in turn)
    __shared__ RowSlot s_rows[3];
    int64_t q_next = 0;  // thread 0's processing index
    if (tid == 0) {
        q_next = first_ticket(p);
        int b0 = 0, len0 = 0;
        s_rows[0].r = find_read_row(p, rows, q_next, b0, len0);
        s_rows[0].b = b0;
        s_rows[0].len = len0;
        publish_next_row(p, rows, q_next, s_rows[1]);
    }
    __syncthreads();
    int b = 0, new_len = 0, par = 0, rslot = 0;
    int64_t r = read_row_slot(s_rows[0], b, new_len);
    int bn = 0, lenn = 0;
    int64_t rn = read_row_slot(s_rows[1], bn, lenn);
    if (r < rows) {
        load_windows(r);
        if (seg == 0 && rn < rows) stage_windows(rn);
    }
    while (r < rows) {
        const int slot2 = rslot == 0 ? 2 : rslot - 1;  // (rslot + 2) % 3
        if (tid == 0) publish_next_row(p, rows, q_next, s_rows[slot2]);
        const bool mask_eos = new_len < min_length_of(p, b);
        const uint16_t* row = static_cast<const uint16_t*>(p.x) + r * V;
        const int sh = static_cast<int>((r * static_cast<int64_t>(V)) & 1);
        // Opaque copies per row: what the unrolled code derives from them is
        // recomputed per row instead of being hoisted out of the row loop
        // into (spilled) registers.
        int nwin_r = nwin, V_r = V, tr = t, sh_r = sh;
        asm volatile("" : "+s"(nwin_r), "+s"(V_r), "+s"(sh_r));
        asm volatile("" : "+v"(tr));

        // ---- padding, row maximum, flag, group maxima ----
        // registers past the segment's windows, and positions outside the
        // row, hold -inf (term 0, never a survivor)
        uint32_t gmax[kGroups], gmin[kGroups];
        uint32_t umax = 0;
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            gmax[g] = 0x80008000u;
            gmin[g] = kPad2;
        }
#pragma unroll
        for (int i = 0; i < kWin; ++i) {
            uint32_t R = reg[i];
            const int w = w_begin + i;
            if (i >= nwin_r) {
                R = kPad2;
            } else if ((w == 0 && sh_r != 0) || 256 * (w + 1) > V_r + sh_r) {
                const int v0 = 256 * w + 2 * tr - sh_r;
                const bool lo_out = v0 < 0 || v0 >= V_r;
                const bool hi_out = v0 + 1 >= V_r;
                R = (lo_out ? kPad : (R & 0xffffu)) | (hi_out ? (kPad << 16) : (R & 0xffff0000u));
            }
            reg[i] = R;
            const int g = i / kGroupRegs;
            gmax[g] = pk_max_i16(gmax[g], R);
            gmin[g] = pk_min_i16(gmin[g], R);
            umax = pk_max_u16(umax, R);
        }

        // (keys: key16 of the largest pattern of a group, per half the largest
        // non-negative pattern, else the smallest signed one)
        int gkey[kGroups];
        int tkey = -32768;
        uint32_t allmax = 0x80008000u;
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            int best = -32768;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int16_t smax = static_cast<int16_t>(gmax[g] >> (16 * h));
                const int16_t smin = static_cast<int16_t>(gmin[g] >> (16 * h));
                const int kk = key16(static_cast<uint16_t>(smax >= 0 ? smax : smin));
                best = max(best, kk);
            }
            gkey[g] = best;
            tkey = max(tkey, best);
            allmax = pk_max_i16(allmax, gmax[g]);
        }
        const bool bad = static_cast<int16_t>(allmax & 0xffffu) >= kPosInf ||
                         static_cast<int16_t>(allmax >> 16) >= kPosInf || (umax & 0xffffu) > kNegInf ||
                         (umax >> 16) > kNegInf;
        if (M > 0) atomicAdd(&s_hist1[(tkey + 32768) >> 8], 1);
        int wkey = tkey;
        for (int off = 32; off > 0; off >>= 1) wkey = max(wkey, __shfl_xor(wkey, off));
        const bool wbad = __any(bad);
        if (l == 0) {
            s_wkey[wave] = wkey;
            s_wbad[wave] = wbad ? 1 : 0;
        }
        lds_barrier();
        int bnn = 0, lennn = 0;
        const int64_t rnn = read_row_slot(s_rows[slot2], bnn, lennn);  // published before the barrier

        int mkey = -32768;
        bool any_bad = false;
#pragma unroll
        for (int w = 0; w < kPipeThreads / 64; ++w) {
            mkey = max(mkey, s_wkey[w]);
            any_bad = any_bad || s_wbad[w] != 0;
        }
        float m = pattern_value<DT>(key_pattern(mkey));
        if (any_bad) {
            // NaN or +inf in the row: the maximum is over x < +inf (reference
            // src/kernels_scalar.cpp:48-56). No shortlist is kept for such a row.
            // (rare: the segment is re-read from the row, which keeps the
            // register file free of a second unrolled pass)
            float lm = -kInf;
            for (int i = 0; i < nwin_r; ++i) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int v = 256 * (w_begin + i) + 2 * t + h - sh;
                    const float x = (v >= 0 && v < V) ? load_one<DT>(row, v) : -kInf;
                    if (x < kInf && x > lm) lm = x;
                }
            }
            lds_barrier();  // every read of the wavefront keys above is done
            const float wm = wave_max(lm);
            if (l == 0) s_wkey[wave] = static_cast<int>(f32_bits(wm));
            lds_barrier();
            m = -kInf;
#pragma unroll
            for (int w = 0; w < kPipeThreads / 64; ++w) m = fmaxf(m, bits_f32(static_cast<uint32_t>(s_wkey[w])));
        }

        // theta: the M-th largest of the 512 thread maxima (at least M
        // elements are >= it), radix-selected on the 16-bit keys
        const bool select = M > 0 && !any_bad;
        int b1 = 0, above1 = 0;
        if (select) {
            hist_select(s_hist1, M, l, b1, above1);
            if (((tkey + 32768) >> 8) == b1) atomicAdd(&s_hist2[(tkey + 32768) & 255], 1);
        }
        int ulo = 0;
        const bool do_lse = LOGITS && m > -kInf;
        const bool use_table = DT == 2 && do_lse && table_fits(m, ulo);
        if (use_table) {
            const uint32_t mp = f32_bits(m) >> 16;
            for (int s = tid; s < 2 * kLutHalf; s += kPipeThreads) {
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
        lds_barrier();
        int tk = -32768;  // key(theta)
        if (select) {
            int b2 = 0, above2 = 0;
            hist_select(s_hist2, M - above1, l, b2, above2);
            tk = ((b1 << 8) | b2) - 32768;
        }
        if (tid < 256) s_hist1[tid] = 0;  // every wavefront has its b1
        const float theta = M > 0 ? (select ? pattern_value<DT>(key_pattern(tk)) : -kInf) : kInf;
        const bool full = M > 0 && !(theta > -kInf);  // no shortlist: every element would survive

        // ---- registers holding x >= theta (groups whose maximum reaches it) ----
        // A packed key test marks them (a superset: keys >= key(theta) - 1, so
        // -0 and +0 both pass); their elements are re-read from the row.
        uint32_t hm[(kWin + 31) / 32] = {};
        if (M > 0 && !full) {
            const int tk1 = tk > -32768 ? tk - 1 : tk;
            const uint32_t tk2 = static_cast<uint32_t>(static_cast<uint16_t>(tk1)) * 0x10001u;
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
                if (gkey[g] >= tk1) {
#pragma unroll
                    for (int q = 0; q < kGroupRegs; ++q) {
                        const int k = g * kGroupRegs + q;
                        const uint32_t R = reg[k];
                        const uint32_t key = R ^ (pk_sign_fill_i16(R) & 0x7fff7fffu);
                        const uint32_t d = pk_sub_sat_i16(key, tk2) & 0x80008000u;
                        hm[k >> 5] |= (d != 0x80008000u ? 1u : 0u) << (k & 31);
                    }
                }
            }
        }
        float* s_acc = s_acc2 + 256 * par;
        int* s_count = s_count2 + par;
        uint64_t* s_key = s_key2 + kSurvivorCap * par;
        float* s_x = s_x2 + kSurvivorCap * par;
        auto push_hits = [&]() {
#pragma unroll
            for (int w = 0; w < (kWin + 31) / 32; ++w) {
                uint32_t bits = hm[w];
                while (bits != 0u) {
                    const int k = 32 * w + __builtin_ctz(bits);
                    bits &= bits - 1u;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int v = 256 * (w_begin + k) + 2 * t + h - sh;
                        const float x = (v >= 0 && v < V) ? load_one<DT>(row, v) : -kInf;
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

        // ---- the lane chains, segment by segment; the next rows stream in ----
        // Step g: segment g folds its windows (continuing the sums segment
        // g - 1 left in s_acc); segment g - 1 loads its windows of the next
        // row; segments 1..3 record their survivors at step 0, segment 0 at
        // step 2, after it has taken the next row from the staging area at
        // step 1 and before it refills the area (two rows ahead) at step 3.
        const int lane_lo = (2 * t - sh) & 255, lane_hi = (2 * t + 1 - sh) & 255;
#pragma unroll 1
        for (int g = 0; g <= kSegs; ++g) {
            if (seg == g && do_lse) {
                float a0 = g == 0 ? 0.0f : s_acc[lane_lo];
                float a1 = g == 0 ? 0.0f : s_acc[lane_hi];
                if (use_table) {
                    // table index of a pattern: magnitude - (u_lo - 1) saturated
                    // at 0 (slot 0) and clamped to 4095, plus 4096 for negative
                    // x; the two halves of a register at once
                    const uint32_t base2 = static_cast<uint32_t>(ulo - 1) * 0x10001u;
                    auto lookup = [&](int k, float& lo, float& hi) {
                        const uint32_t R = reg[k];
                        uint32_t idx = pk_sub_sat_u16(R & 0x7fff7fffu, base2);
                        idx = pk_min_u16(idx, 0x0fff0fffu);
                        idx |= (R >> 3) & 0x10001000u;
                        const uint32_t addr = pk_shl2_u16(idx);
                        lo = lut[(addr & 0xffffu) >> 2];
                        hi = lut[addr >> 18];
                    };
                    // blocks of kBlk registers; the lookups of block b + 1 are
                    // in flight while block b is added in order (padding
                    // registers add zeros)
                    float cur[2 * kBlk], nxt[2 * kBlk];
#pragma unroll
                    for (int q = 0; q < kBlk; ++q) lookup(q, cur[2 * q], cur[2 * q + 1]);
#pragma unroll
                    for (int k0 = 0; k0 < kWin; k0 += kBlk) {
                        __builtin_amdgcn_sched_barrier(0);
                        if (k0 + kBlk < kWin) {
#pragma unroll
                            for (int q = 0; q < kBlk; ++q) lookup(k0 + kBlk + q, nxt[2 * q], nxt[2 * q + 1]);
                        }
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int q = 0; q < kBlk; ++q) {
                            a0 = a0 + cur[2 * q];
                            a1 = a1 + cur[2 * q + 1];
                        }
#pragma unroll
                        for (int q = 0; q < 2 * kBlk; ++q) cur[q] = nxt[q];
                    }
                } else {
                    // Cephes terms of the finite elements, re-read from the
                    // row (rows the table does not cover, and 16-bit floats)
                    for (int i = 0; i < nwin_r; ++i) {
                        const int v = 256 * (w_begin + i) + 2 * t - sh;
                        const float x0 = (v >= 0 && v < V) ? load_one<DT>(row, v) : -kInf;
                        const float x1 = v + 1 < V ? load_one<DT>(row, v + 1) : -kInf;
                        if (x0 < kInf && x0 > -kInf) a0 = a0 + exp_nonpositive(x0 - m);
                        if (x1 < kInf && x1 > -kInf) a1 = a1 + exp_nonpositive(x1 - m);
                    }
                }
                s_acc[lane_lo] = a0;
                s_acc[lane_hi] = a1;
            }
            if (g == 0 && seg != 0) push_hits();
            if (seg == 0) {
                if (g == 0 && rn < rows) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the staged row is in
                if (g == 1 && wave == 0 && pend) finish_pending();
                if (g == 1 && rn < rows) {
#pragma unroll
                    for (int i = 0; i < kWin; ++i) reg[i] = stage[64 * i + l];
                }
                if (g == 2) {
                    s_hist2[t] = 0;  // every wavefront has read its b2 (barriers since)
                    s_hist2[t + 128] = 0;
                    push_hits();
                }
                if (g == 3 && rnn < rows) stage_windows(rnn);
            }
            if (seg >= 1 && g == seg + 1 && rn < rows) load_windows(rn);
            lds_barrier();
        }

        if (wave == 0) {
            pend = true;
            pend_r = r;
            pend_m = m;
            pend_theta = theta;
            pend_bad = any_bad;
            pend_lse = do_lse;
            pend_mask = mask_eos;
            pend_full = full;
            pend_b = b;
            pend_par = par;
        }
        par ^= 1;
        rslot = rslot == 2 ? 0 : rslot + 1;
        r = rn;
        b = bn;
        new_len = lenn;
        rn = rnn;
        bn = bnn;
        lenn = lennn;
    }
    if (wave == 0 && pend) finish_pending();
}

int g_pipe_cu_count[64];

// Windows per segment of a vocabulary.
int pipe_windows(int V) { return ((V + 256) / 256 + kSegs - 1) / kSegs; }

template <int DT, bool LOGITS>
hipError_t launch_pipe(const DecodeParams& p, int64_t rows, int device, hipStream_t stream) {
    // one workgroup per CU, less the CUs left to an overlapped select pass
    const int64_t cus = g_pipe_cu_count[device] - p.reserve_cus > 0 ? g_pipe_cu_count[device] - p.reserve_cus : 1;
    const int64_t grid = rows < cus ? rows : cus;
    const dim3 g(static_cast<unsigned>(grid)), blk(kPipeThreads);
    const int P = pipe_windows(p.V);
    if (P <= 64) hipLaunchKernelGGL((row_pipe_kernel<DT, LOGITS, 64>), g, blk, 0, stream, p, rows);
    else if (P <= 128) hipLaunchKernelGGL((row_pipe_kernel<DT, LOGITS, 128>), g, blk, 0, stream, p, rows);
    else hipLaunchKernelGGL((row_pipe_kernel<DT, LOGITS, kMaxWin>), g, blk, 0, stream, p, rows);
    return hipGetLastError();
}

}  // namespace

bool row_pipe_eligible(const DecodeParams& p) {
    if (p.dtype != 1 && p.dtype != 2) return false;
    if (reinterpret_cast<uintptr_t>(p.x) % 4 != 0) return false;
    if (pipe_windows(p.V) > kMaxWin) return false;
    return p.M <= 256;
}

hipError_t launch_row_pipe(const DecodeParams& p, int64_t rows, hipStream_t stream) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    if (g_pipe_cu_count[device] == 0) {
        int cus = 0;
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
        if (e != hipSuccess) return e;
        g_pipe_cu_count[device] = cus > 0 ? cus : 1;
    }
    if (p.from_logits) return p.dtype == 2 ? launch_pipe<2, true>(p, rows, device, stream)
                                           : launch_pipe<1, true>(p, rows, device, stream);
    return p.dtype == 2 ? launch_pipe<2, false>(p, rows, device, stream)
                        : launch_pipe<1, false>(p, rows, device, stream);
}

}  // namespace dbs_hip
