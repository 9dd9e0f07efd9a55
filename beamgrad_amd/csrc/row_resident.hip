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
//   * each wavefront loads its 64 lanes in chunks of 8 stripes, all in flight
//     at once: one 16-byte buffer load per lane brings a chunk (1 KB) into the
//     registers it will occupy; a pass through a 1 KB LDS slot (one write, two
//     transposing reads) gives each lane its own elements of the chunk;
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

#include "row_helpers.hpp"

namespace dbs_hip {

namespace {

constexpr int kResThreads = 512;                 // two segments of the 256 lanes
constexpr int kResRegs = 152;                    // packed element pairs per thread
constexpr int kResChunks = kResRegs / 4;         // 8-stripe chunks per thread
constexpr int kResGroups = 4;                    // register groups with their own maxima
constexpr int kResGroupRegs = kResRegs / kResGroups;
constexpr int kMaxStripes = 2 * 8 * kResChunks;  // 608 stripes: V <= 155648

// LDS, as separate arrays.
constexpr int kResLds = 2 * kLutHalf * 4 + 8 * 1024 + 256 * 4 + kSurvivorCap * 12 + 2 * 256 * 4 + 64 + 16;
static_assert(kResLds <= 160 * 1024, "LDS of the resident row pass");

template <int DT, bool LOGITS>
__global__ __launch_bounds__(kResThreads) void row_resident_kernel(DecodeParams p, int64_t rows) {
    __shared__ __attribute__((aligned(16))) float lut[2 * kLutHalf];
    __shared__ __attribute__((aligned(16))) unsigned char s_stage[8 * 1024];
    __shared__ float s_acc[256];
    __shared__ uint64_t s_key[kSurvivorCap];
    __shared__ float s_x[kSurvivorCap];
    __shared__ __attribute__((aligned(16))) int s_hist[2 * 256];
    __shared__ int s_wave[16];
    __shared__ int s_count_arr[1];
    int* s_hist1 = s_hist;
    int* s_hist2 = s_hist + 256;
    int* s_wkey = s_wave;
    int* s_wbad = s_wave + 8;
    int* s_count = s_count_arr;

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
    unsigned char* stage = s_stage + wave * 1024;

    if (tid == 0) *s_count = 0;
    if (tid < 256) {
        s_hist1[tid] = 0;
        s_hist2[tid] = 0;
    }
    __syncthreads();

    // Wavefront kFinisher (the first of segment 1) finishes row r (lane tree,
    // shortlist, RowInfo; counted done for the overlapped decode) at the
    // start of the next row, while its part of that row is still arriving.
    constexpr int kFinisher = 4;
    bool pend = false;
    int64_t pend_r = 0;
    float pend_m = 0.0f, pend_theta = 0.0f;
    bool pend_bad = false, pend_lse = false, pend_mask = false, pend_full = false;
    int pend_b = 0;
    auto finish_pending = [&]() {
        float lse = 0.0f;
        if (LOGITS) {
            if (pend_lse) {
                float a[4];
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) a[e2] = s_acc[4 * l + e2];
                lse = logsumexp_from(pend_m, lane_tree_sum(a, l));
            } else {
                lse = -kInf;
            }
        }
        const int n = pend_full ? kSurvivorCap + 1 : *s_count;
        finish_row_wave<LOGITS, true>(p, pend_r, lse, pend_theta, pend_bad, s_key, s_x, n, l, pend_b, pend_mask);
        wave_sync();
        if (l == 0) *s_count = 0;
        pend = false;
    };

    // byte offset in the segment of this lane's 16 bytes of chunk 0 (stripe
    // l/8 of the segment, lanes 64 wv + 8 (l % 8) ..); chunk c adds the
    // scalar 4096 c
    auto lane_offset = [&]() -> int {
        int lr = l;
        asm volatile("" : "+v"(lr));
        return 2 * (256 * (lr >> 3) + 64 * wv + 8 * (lr & 7));
    };

    // The row sequence: every wavefront steps through its workgroup's rows
    // by itself (in scalar registers); with tickets, thread 0 takes them and
    // publishes them in LDS slots by row parity.
    __shared__ RowSlot s_rows[2];
    const bool tickets = p.row_ticket != nullptr;
    auto next_read_row = [&](int64_t rr, int& b_out, int& len_out) -> int64_t {
        while (rr < rows && !row_is_read(p, rr, b_out, len_out)) rr += gridDim.x;
        b_out = __builtin_amdgcn_readfirstlane(b_out);
        len_out = __builtin_amdgcn_readfirstlane(len_out);
        const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(rr));
        const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(rr) >> 32));
        return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
    };
    int64_t q_next = 0;  // thread 0's processing index (tickets)
    int b = 0, new_len = 0, par = 0;
    int64_t r = rows;
    if (tickets) {
        if (tid == 0) {
            q_next = first_ticket(p);
            int b0 = 0, len0 = 0;
            s_rows[0].r = find_read_row(p, rows, q_next, b0, len0);
            s_rows[0].b = b0;
            s_rows[0].len = len0;
        }
        __syncthreads();
        r = read_row_slot(s_rows[0], b, new_len);
    } else {
        r = next_read_row(blockIdx.x, b, new_len);
    }
    // Chunk c (8 stripes x this wavefront's 64 lanes): lane l loads the 16
    // bytes of stripe 8c + l/8, lanes 64 wv + 8 (l % 8) .. into the four
    // registers the chunk will occupy. Every chunk is in flight at once; the
    // buffer view covers exactly the segment's stripes inside the row, so
    // groups past it read zeros without touching memory, and are replaced by
    // padding; a row index past the last gives an empty view. Each segment
    // loads its part of the next row as soon as its chain has passed its
    // registers: segment 0 while segment 1 folds, segment 1 at the row's end.
    uint32_t reg[kResRegs];
    auto row_view = [&](int64_t rr) {
        int V_r = V;
        asm volatile("" : "+s"(V_r));
        const bool any = rr < rows;
        const uint16_t* rrow = static_cast<const uint16_t*>(p.x) + (any ? rr : 0) * V_r;
        const int seg_bytes = any ? max(0, 2 * min(V_r, 256 * (s_begin + per)) - 512 * s_begin) : 0;
        return row_buffer(rrow + 256 * s_begin, seg_bytes);
    };
    auto issue_chunk = [&](const __amdgpu_buffer_rsrc_t& rs, int voff, int c) {
        const v4u32 q = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 4096 * c, 0);
        reg[4 * c] = q.x;
        reg[4 * c + 1] = q.y;
        reg[4 * c + 2] = q.z;
        reg[4 * c + 3] = q.w;
    };
    auto issue_loads = [&](int64_t rr) {
        const __amdgpu_buffer_rsrc_t rs = row_view(rr);
        const int voff = lane_offset();
#pragma unroll
        for (int c = 0; c < kResChunks; ++c) issue_chunk(rs, voff, c);
    };
    if (r < rows) issue_loads(r);
    while (r < rows) {
        int bn = 0, lenn = 0;
        int64_t rn = rows;
        if (tickets) {
            if (tid == 0) publish_next_row(p, rows, q_next, s_rows[par ^ 1]);
        } else {
            rn = next_read_row(r + gridDim.x, bn, lenn);
        }
        // the next row (with tickets: published before this row's first barrier)
        auto next_row = [&]() -> int64_t {
            if (!tickets) return rn;
            int bt = 0, lt = 0;
            return read_row_slot(s_rows[par ^ 1], bt, lt);
        };
        const bool mask_eos = new_len < min_length_of(p, b);
        const uint16_t* row = static_cast<const uint16_t*>(p.x) + r * V;
        // Opaque copies per row: everything the unrolled load derives from
        // them is recomputed per row instead of being hoisted out of the row
        // loop into (spilled) registers.
        int V_r = V, jr = j, lr = l;
        asm volatile("" : "+s"(V_r));
        asm volatile("" : "+v"(jr), "+v"(lr));
        if (wave == kFinisher && pend) finish_pending();

        // ---- the row's segment in registers (loaded during the previous
        // row, see issue_loads), transposed to lanes ----
        // registers past the segment's chunks hold -inf pairs (term 0, never
        // a survivor), so the chain below runs over all of them unguarded
        uint32_t gmax[kResGroups], gmin[kResGroups];
        uint32_t umax = 0;
#pragma unroll
        for (int g = 0; g < kResGroups; ++g) {
            gmax[g] = 0x80008000u;
            gmin[g] = kPad | (kPad << 16);
        }
        // Software-pipelined: chunk c + 1's transpose is issued before chunk
        // c's results are used. Chunks past the segment (zeros from the view)
        // and elements past the row become padding.
        const int seg_end = min(V_r, 256 * (s_begin + per));  // elements of the segment end here
        uint32_t Tn[4];
        transpose_chunk(stage, lr, reg[0], reg[1], reg[2], reg[3], Tn);
#pragma unroll
        for (int c = 0; c < kResChunks; ++c) {
            uint32_t R4[4] = {Tn[0], Tn[1], Tn[2], Tn[3]};
            if (c + 1 < kResChunks)
                transpose_chunk(stage, lr, reg[4 * c + 4], reg[4 * c + 5], reg[4 * c + 6], reg[4 * c + 7], Tn);
            const int sb = s_begin + 8 * c;
            if (256 * (sb + 8) > seg_end) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const bool lo_out = 256 * (sb + 2 * q) + jr >= seg_end;
                    const bool hi_out = 256 * (sb + 2 * q + 1) + jr >= seg_end;
                    R4[q] = (lo_out ? kPad : (R4[q] & 0xffffu)) | (hi_out ? (kPad << 16) : (R4[q] & 0xffff0000u));
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int k = 4 * c + q;
                const uint32_t R = R4[q];
                reg[k] = R;
                const int g = k / kResGroupRegs;
                gmax[g] = pk_max_i16(gmax[g], R);
                gmin[g] = pk_min_i16(gmin[g], R);
                umax = pk_max_u16(umax, R);
            }
        }

        // ---- row maximum, flag, group keys; the key histogram for theta ----
        // (keys: key16 of the largest pattern of a group, per half the largest
        // non-negative pattern, else the smallest signed one)
        int gkey[kResGroups];
        int tkey = -32768;
        uint32_t allmax = 0x80008000u;
#pragma unroll
        for (int g = 0; g < kResGroups; ++g) {
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

        int mkey = -32768;
        bool any_bad = false;
#pragma unroll
        for (int w = 0; w < kResThreads / 64; ++w) {
            mkey = max(mkey, s_wkey[w]);
            any_bad = any_bad || s_wbad[w] != 0;
        }
        float m = pattern_value<DT>(key_pattern(mkey));
        if (any_bad) {
            // NaN or +inf in the row: the maximum is over x < +inf (reference
            // src/kernels_scalar.cpp:48-56), so re-read the segment for it.
            // No shortlist is kept for such a row.
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
            lds_barrier();  // every read of the wavefront keys above is done
            const float wm = wave_max(lm);
            if (l == 0) s_wkey[wave] = static_cast<int>(f32_bits(wm));
            lds_barrier();
            m = -kInf;
#pragma unroll
            for (int w = 0; w < kResThreads / 64; ++w) m = fmaxf(m, bits_f32(static_cast<uint32_t>(s_wkey[w])));
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
            // the 8192 slots, 16 per thread (slots tid + 512 i: the negative
            // half from i = 8), evaluated without branches; slots past the
            // row's range hold 0
            const uint32_t mp = f32_bits(m) >> 16;
            const float em = exp_nonpositive(-m);
#pragma unroll
            for (int i = 0; i < 2 * kLutHalf / kResThreads; ++i) {
                const bool neg = i >= kLutHalf / kResThreads;
                const int k = tid + kResThreads * (i % (kLutHalf / kResThreads));
                const int u = ulo - 1 + k;
                const bool valid = u < 0x7f80 && (neg || u <= static_cast<int>(mp));
                const float x = bf16_to_f32(static_cast<uint16_t>((neg ? 0x8000 : 0) | (valid ? u : 0)));
                const float t = exp_nonpositive_nb(x - m);
                lut[(neg ? kLutHalf : 0) + k] = k == 0 ? em : (valid ? t : 0.0f);
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
        // -0 and +0 both pass); their elements are re-read from the row, which
        // is still in cache, while the other segment folds its lanes.
        uint32_t hm[(kResRegs + 31) / 32] = {};
        if (M > 0 && !full) {
            const int tk1 = tk > -32768 ? tk - 1 : tk;
            const uint32_t tk2 = static_cast<uint32_t>(static_cast<uint16_t>(tk1)) * 0x10001u;
#pragma unroll
            for (int g = 0; g < kResGroups; ++g) {
                if (gkey[g] >= tk1) {
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
        // Their elements, re-read from the row (in cache): the loads of up to
        // four marked registers are in flight at once, then each element
        // reaching theta goes to the LDS list (banned and masked tokens are
        // dropped when the row is finished).
        auto push_hits = [&]() {
#pragma unroll
            for (int w = 0; w < (kResRegs + 31) / 32; ++w) {
                uint32_t bits = hm[w];
                while (bits != 0u) {
                    int ks[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        ks[u] = bits != 0u ? 32 * w + __builtin_ctz(bits) : -1;
                        bits &= bits - 1u;
                    }
                    float xs[8];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const int v = 256 * (s_begin + 2 * ks[u] + h) + j;
                            const bool ok = ks[u] >= 0 && v < V;
                            const float xv = load_one<DT>(row, ok ? v : 0);  // in bounds either way
                            xs[2 * u + h] = ok ? xv : -kInf;
                        }
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const float x = xs[2 * u + h];
                            if (x >= theta && x < kInf && x > -kInf) {
                                const int slot = atomicAdd(s_count, 1);
                                if (slot < kSurvivorCap) {
                                    s_key[slot] = survivor_key(x, 256 * (s_begin + 2 * ks[u] + h) + j);
                                    s_x[slot] = x;
                                }
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
            lds_barrier();
        }
        bool loaded = false;  // the next row's loads are issued
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
                    lo = lut[(addr & 0xffffu) >> 2];
                    hi = lut[addr >> 18];
                };
                // blocks of kBlk registers; the lookups of block b + 1 are in
                // flight while block b is added in order
                // (a block is one loaded chunk: once its lookups are issued,
                // its registers take the same chunk of the next row)
                constexpr int kBlk = 4;
                static_assert(kBlk == 4, "a lookup block is one chunk");
                const __amdgpu_buffer_rsrc_t rs_next = row_view(next_row());
                const int voff_next = lane_offset();
                float cur[2 * kBlk], nxt[2 * kBlk];
#pragma unroll
                for (int q = 0; q < kBlk; ++q) lookup(q, cur[2 * q], cur[2 * q + 1]);
                issue_chunk(rs_next, voff_next, 0);
#pragma unroll
                for (int k0 = 0; k0 < kResRegs; k0 += kBlk) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (k0 + kBlk < kResRegs) {
#pragma unroll
                        for (int q = 0; q < kBlk; ++q) lookup(k0 + kBlk + q, nxt[2 * q], nxt[2 * q + 1]);
                        issue_chunk(rs_next, voff_next, k0 / kBlk + 1);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int q = 0; q < 2 * kBlk; ++q) acc = acc + cur[q];
#pragma unroll
                    for (int q = 0; q < 2 * kBlk; ++q) cur[q] = nxt[q];
                }
                loaded = true;
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
            lds_barrier();
            s_hist2[tid] = 0;  // every wavefront has read its b2
            push_hits();
        }
        if (!loaded) issue_loads(next_row());
        lds_barrier();

        if (wave == kFinisher) {
            pend = true;
            pend_r = r;
            pend_m = m;
            pend_theta = theta;
            pend_bad = any_bad;
            pend_lse = do_lse;
            pend_mask = mask_eos;
            pend_full = full;
            pend_b = b;
        }
        if (tickets) {
            r = read_row_slot(s_rows[par ^ 1], b, new_len);  // published before this row's first barrier
            par ^= 1;
        } else {
            r = rn;
            b = bn;
            new_len = lenn;
        }
    }
    if (wave == kFinisher && pend) finish_pending();
}

int g_cu_count[64];

template <int DT, bool LOGITS>
hipError_t launch_resident(const DecodeParams& p, int64_t rows, int device, hipStream_t stream) {
    // one workgroup per CU, less the CUs left to an overlapped select pass
    const int64_t cus = g_cu_count[device] - p.reserve_cus > 0 ? g_cu_count[device] - p.reserve_cus : 1;
    const int64_t grid = rows < cus ? rows : cus;
    hipLaunchKernelGGL((row_resident_kernel<DT, LOGITS>), dim3(static_cast<unsigned>(grid)), dim3(kResThreads), 0,
                       stream, p, rows);
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
