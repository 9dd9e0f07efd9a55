// SPDX-License-Identifier: MIT
//
// Row pass for bfloat16 logits rows that keeps each row on chip and keeps
// both wavefronts of every SIMD busy.
//
// The logsumexp of the reference folds exp(x - max) into 256 lanes (lane j =
// v mod 256, increasing v; reference src/kernels_scalar.cpp:48-66): each
// lane's sum is one sequential chain, and the row maximum is needed before
// its first term. One 512-thread workgroup per CU is persistent over rows;
// thread (seg, j) holds lane j of stripes [seg P, seg P + P) of the row (two
// segments of P stripes, stripe s = elements 256 s .. 256 s + 255), two
// stripes per register, so a lane's chain is segment 0's part followed by
// segment 1's. The segments relay each other over a row:
//
//   phase 0  segment 1 transposes its part of the row (arrived in registers
//            during the previous row) and takes its maxima, while one
//            wavefront of segment 0 finishes the previous row (lane tree,
//            logsumexp, shortlist, RowInfo); both segments exchange the
//            maxima: row maximum, NaN/+inf flag, the shortlist threshold (the
//            M-th largest thread maximum) and the row's term table (fixed
//            base, table_fits_fixed);
//   phase A  segment 0 records its chunks that may hold survivors (x >=
//            theta), folds its stripes (the registers hold table slots:
//            extract, look up, add) and streams its part of the next row
//            into the registers it has passed; segment 1 turns its registers
//            into table slots and records its survivor chunks;
//   phase B  segment 1 continues the lane chains over its stripes and
//            streams its part of the next row;
//            segment 0 transposes, keys and converts its part of the next
//            row.
//
// Rows the fixed-base table does not cover (NaN/+inf, maximum below 1 or from
// 127.5 up, every value negative) take their maximum and terms from the row
// in memory with the Cephes evaluation.
#include <hip/hip_runtime.h>

#include <utility>

#include "row_helpers.hpp"

namespace dbs_hip {

namespace {

constexpr int kRlThreads = 512;                 // two segments of the 256 lanes
constexpr int kRlRegs = 152;                    // packed element pairs per thread
constexpr int kRlChunks = kRlRegs / 4;          // 8-stripe chunks per thread
constexpr int kRlStripes = 2 * 8 * kRlChunks;   // 608 stripes: V <= 155648
constexpr uint32_t kBf16NegInf = 0xff80u;
constexpr int kFinisher = 0;                    // the wavefront of segment 0 that finishes rows
constexpr int kRecCap = 32;                     // survivor records per wavefront and row
constexpr int kRlChunksShort = 32;              // chunks per thread for V <= 131072

// f(integral_constant<int, i>) for i = 0 .. N - 1, expanded at compile time:
// every register of the row is indexed with a constant (a loop the compiler
// left rolled would move the whole array to scratch memory).
template <class F, int... I>
__device__ __forceinline__ void unrolled_seq(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void unrolled(F&& f) {
    unrolled_seq(f, std::make_integer_sequence<int, N>{});
}

// Chunks below kMaskFrom are inside the row on every lane of both segments
// (the launch checks it): only the later ones are masked. kChunks 8-stripe
// chunks per thread cover segments of up to 8 kChunks stripes.
template <int kChunks, int kMaskFrom>
__global__ __launch_bounds__(kRlThreads) void row_relay_kernel(DecodeParams p, int64_t rows) {
    constexpr int kRegs = 4 * kChunks;             // packed element pairs per thread
    constexpr int kGroups = (kChunks + 7) / 8;     // chunk keys read eight at a time
    static_assert(kChunks <= kRlChunks && kMaskFrom <= kChunks, "relay chunk range");
    // (the table first: at LDS address 0 its offsets need no base added)
    __shared__ __attribute__((aligned(1024))) float lut[2 * kLutHalf];
    __shared__ __attribute__((aligned(16))) unsigned char s_stage[8 * 1024];
    // chunk keys: thread t's keys of chunks 8 g .. 8 g + 7 at s_ck[g][t]
    __shared__ __attribute__((aligned(16))) int16_t s_ck[kGroups][kRlThreads][8];
    __shared__ float s_acc[2][256];
    __shared__ uint64_t s_key[kSurvivorCap + 2];
    __shared__ float s_x[kSurvivorCap];
    // survivor records by row parity: a lane's chunk (eight patterns as
    // table slots) where its key reaches theta, kRecCap per wavefront
    __shared__ __attribute__((aligned(16))) uint4 s_rec[2][8 * kRecCap];
    __shared__ int s_rtok[2][8 * kRecCap];
    __shared__ __attribute__((aligned(16))) int s_nrec[2][8];
    __shared__ __attribute__((aligned(16))) int s_hist[2 * 256];
    __shared__ int s_wkey[8], s_wbad[8];
    __shared__ RowSlot s_rows[2];
    int* s_hist1 = s_hist;
    int* s_hist2 = s_hist + 256;

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
    unsigned char* stage = s_stage + wave * 1024;

    if (tid < 16) s_nrec[tid >> 3][tid & 7] = 0;
    if (tid < 256) {
        s_hist1[tid] = 0;
        s_hist2[tid] = 0;
    }
    __syncthreads();

    // ---- the row sequence: the workgroup's stride, or tickets published by
    // thread 0 in LDS slots by row parity ----
    const bool tickets = p.row_ticket != nullptr;
    auto next_read_row = [&](int64_t rr, int& b_out, int& len_out) __attribute__((always_inline)) -> int64_t {
        while (rr < rows && !row_is_read(p, rr, b_out, len_out)) rr += gridDim.x;
        b_out = __builtin_amdgcn_readfirstlane(b_out);
        len_out = __builtin_amdgcn_readfirstlane(len_out);
        const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(rr));
        const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(rr) >> 32));
        return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
    };
    // tickets are drawn by a thread of segment 1, which has time to spare
    // in phase 0 (segment 0's wavefront kFinisher is then busy)
    constexpr int kPublisher = 256;
    int64_t q_next = 0;  // the publisher's processing index (tickets)
    int b = 0, new_len = 0, par = 0;
    int64_t r = rows;
    if (tickets) {
        if (tid == kPublisher) {
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

    // ---- loads: chunk c (8 stripes x the wavefront's 64 lanes) of the
    // thread's segment, lane l's 16 bytes of stripe 8c + l/8, lanes 64 wv +
    // 8 (l % 8) .., straight into the registers the chunk will occupy ----
    uint32_t reg[kRegs];
    auto lane_offset = [&]() __attribute__((always_inline)) -> int {
        int lr = l;
        asm volatile("" : "+v"(lr));
        return 2 * (256 * (lr >> 3) + 64 * wv + 8 * (lr & 7));
    };
    auto row_view = [&](int64_t rr) __attribute__((always_inline)) {
        int V_r = V;
        asm volatile("" : "+s"(V_r));
        const bool any = rr < rows;
        const uint16_t* rrow = static_cast<const uint16_t*>(p.x) + (any ? rr : 0) * V_r;
        const int seg_bytes = any ? max(0, 2 * min(V_r, 256 * (s_begin + per)) - 512 * s_begin) : 0;
        return row_buffer(rrow + 256 * s_begin, seg_bytes);
    };
    auto issue_chunk = [&](const __amdgpu_buffer_rsrc_t& rs, int voff, int c) __attribute__((always_inline)) {
        const v4u32 q = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 4096 * c, kRowLoadPolicy);
        reg[4 * c] = q.x;
        reg[4 * c + 1] = q.y;
        reg[4 * c + 2] = q.z;
        reg[4 * c + 3] = q.w;
    };
    auto issue_loads = [&](int64_t rr) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rs = row_view(rr);
        const int voff = lane_offset();
#pragma unroll
        for (int c = 0; c < kChunks; ++c) issue_chunk(rs, voff, c);
    };

    // ---- arrival: the segment's chunks transposed to lanes (a lane's 16
    // bytes past the row, V % 8 == 0, go in as -inf), the thread's packed
    // signed and unsigned pattern maxima, per chunk the largest signed
    // pattern (the chunk's maximum where it is >= +0) in s_ck, and the
    // registers turned into table slots (term_slots) ----
    uint32_t t_smax = 0x80008000u, t_umax = 0u;
    // the lane's loaded 16 bytes of chunk c are past the row from c = c_lim
    // on (element 256 (s_begin + 8 c + l / 8) + 64 wv + 8 (l % 8) >= end)
    auto lane_c_lim = [&]() __attribute__((always_inline)) -> int {
        int lr = l;
        asm volatile("" : "+v"(lr));
        const int end_r = min(V, 256 * (s_begin + per));
        const int first = 256 * (s_begin + (lr >> 3)) + 64 * wv + 8 * (lr & 7);
        int c_lim = (end_r - first + 2047) >> 11;
        asm volatile("" : "+v"(c_lim));
        return c_lim;
    };

    // the maxima of the loaded registers as they are (each thread's values
    // are then 8 lanes of kChunks stripes: any partition of the row serves the
    // row maximum and the shortlist threshold)
    auto keys_loaded = [&]() __attribute__((always_inline)) {
        const int c_lim = lane_c_lim();
        uint32_t smax = 0x80008000u, umax = 0u;
        unrolled<kChunks>([&](auto cc) __attribute__((always_inline)) {
            constexpr int c = decltype(cc)::value;
            uint32_t a = reg[4 * c], b2 = reg[4 * c + 1], c2 = reg[4 * c + 2], d = reg[4 * c + 3];
            if constexpr (c >= kMaskFrom) {
                const bool in = c < c_lim;
                a = in ? a : kBf16NegInf * 0x10001u;
                b2 = in ? b2 : kBf16NegInf * 0x10001u;
                c2 = in ? c2 : kBf16NegInf * 0x10001u;
                d = in ? d : kBf16NegInf * 0x10001u;
            }
            smax = pk_max_i16(smax, pk_max_i16(pk_max_i16(a, b2), pk_max_i16(c2, d)));
            umax = pk_max_u16(umax, pk_max_u16(pk_max_u16(a, b2), pk_max_u16(c2, d)));
            asm volatile("" : "+v"(smax), "+v"(umax));  // chunk by chunk: no masked copies kept
        });
        t_smax = smax;
        t_umax = umax;
    };
    auto arrive = [&]() __attribute__((always_inline)) {
        int lr = l;
        asm volatile("" : "+v"(lr));
        const int c_lim = lane_c_lim();
        // chunk c's registers masked in place just before its transpose
        auto mask_chunk = [&](auto cc) __attribute__((always_inline)) {
            constexpr int c = decltype(cc)::value;
            if constexpr (c < kMaskFrom) return;
            const bool in = c < c_lim;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                reg[4 * c + q] = in ? reg[4 * c + q] : kBf16NegInf * 0x10001u;
                asm volatile("" : "+v"(reg[4 * c + q]));
            }
        };
        uint32_t smax = 0x80008000u, umax = 0u;
        // two chunks' transposes in flight (chunk c's values in T[c % 2]);
        // one slot serves both: a wavefront's LDS operations run in order
        uint32_t T[2][4];
        uint32_t ckp[4];  // the keys of eight chunks, two per register, written together
        mask_chunk(std::integral_constant<int, 0>{});
        transpose_chunk(stage, lr, reg[0], reg[1], reg[2], reg[3], T[0]);
        mask_chunk(std::integral_constant<int, 1>{});
        transpose_chunk(stage, lr, reg[4], reg[5], reg[6], reg[7], T[1]);
        unrolled<kChunks>([&](auto cc) __attribute__((always_inline)) {
            constexpr int c = decltype(cc)::value;
            const uint32_t R4[4] = {T[c & 1][0], T[c & 1][1], T[c & 1][2], T[c & 1][3]};
            if constexpr (c + 2 < kChunks) {
                mask_chunk(std::integral_constant<int, c + 2>{});
                transpose_chunk(stage, lr, reg[4 * c + 8], reg[4 * c + 9], reg[4 * c + 10], reg[4 * c + 11], T[c & 1]);
            }
            const uint32_t kc = pk_max_i16(pk_max_i16(R4[0], R4[1]), pk_max_i16(R4[2], R4[3]));
            smax = pk_max_i16(smax, kc);
            umax = pk_max_u16(umax, pk_max_u16(pk_max_u16(R4[0], R4[1]), pk_max_u16(R4[2], R4[3])));
            const uint32_t ck = static_cast<uint32_t>(max(static_cast<int>(static_cast<int16_t>(kc & 0xffffu)),
                                                          static_cast<int>(static_cast<int16_t>(kc >> 16)))) & 0xffffu;
            if constexpr ((c & 1) == 0) ckp[(c & 7) >> 1] = ck | 0x80000000u;  // (the odd chunk's key replaces -32768)
            else ckp[(c & 7) >> 1] = (ckp[(c & 7) >> 1] & 0xffffu) | (ck << 16);
            if constexpr ((c & 7) == 7 || c + 1 == kChunks) {
#pragma unroll
                for (int u = ((c & 7) >> 1) + 1; u < 4; ++u) ckp[u] = 0x80008000u;  // chunks past the last
                *reinterpret_cast<uint4*>(&s_ck[c >> 3][tid][0]) = make_uint4(ckp[0], ckp[1], ckp[2], ckp[3]);
            }
            asm volatile("" : "+v"(smax), "+v"(umax));  // the maxima taken here: the patterns die here
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                reg[4 * c + q] = term_slots(R4[q]);
                asm volatile("" : "+v"(reg[4 * c + q]));
            }
        });
        t_smax = smax;
        t_umax = umax;
    };

    // ---- the segment's part of a lane chain from the table slots; the
    // registers take the next row's chunks as the chain passes them ----
    auto chain_table = [&](float acc, int64_t rn) __attribute__((always_inline)) -> float {
        const unsigned char* lut_bytes = reinterpret_cast<const unsigned char*>(lut);
        // the two slots' byte offsets, each with one shift of its 16-bit half
        // (SDWA word select; the compiler picks it for the upper half only)
        const uint32_t two = 2u;
        auto lookup = [&](int k, float& lo, float& hi) __attribute__((always_inline)) {
            const uint32_t A = reg[k];
            uint32_t lo_off;
            asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_0"
                : "=v"(lo_off)
                : "v"(two), "v"(A));
            lo = *reinterpret_cast<const float*>(lut_bytes + lo_off);
            hi = *reinterpret_cast<const float*>(lut_bytes + ((A >> 16) << 2));
        };
        const __amdgpu_buffer_rsrc_t rs_next = row_view(rn);
        const int voff_next = lane_offset();
        float cur[8], nxt[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) lookup(q, cur[2 * q], cur[2 * q + 1]);
        issue_chunk(rs_next, voff_next, 0);
        unrolled<kChunks>([&](auto cc) __attribute__((always_inline)) {
            constexpr int k0 = 4 * decltype(cc)::value;
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (k0 + 4 < kRegs) {
#pragma unroll
                for (int q = 0; q < 4; ++q) lookup(k0 + 4 + q, nxt[2 * q], nxt[2 * q + 1]);
                issue_chunk(rs_next, voff_next, k0 / 4 + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < 8; ++q) acc = acc + cur[q];
            asm volatile("" : "+v"(acc));  // the terms are added here, not sunk past the chain
#pragma unroll
            for (int q = 0; q < 8; ++q) cur[q] = nxt[q];
        });
        return acc;
    };
    // Cephes terms from the row in memory (its lines are cached)
    auto chain_memory = [&](float acc, float m, const uint16_t* row) __attribute__((always_inline)) -> float {
        for (int s = s_begin; s < s_begin + 8 * nch; s += 8) {
            float xs[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int v = 256 * (s + u) + j;
                xs[u] = v < V ? load_one<2>(row, v) : -kInf;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (xs[u] < kInf && xs[u] > -kInf) acc = acc + exp_nonpositive(xs[u] - m);
        }
        return acc;
    };
    // the row maximum over x < +inf from the row in memory (both segments
    // together; every thread of the workgroup calls it)
    auto memory_max = [&](const uint16_t* row) __attribute__((always_inline)) -> float {
        float lm = -kInf;
        for (int s = s_begin; s < s_begin + 8 * nch; s += 8) {
            float xs[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int v = 256 * (s + u) + j;
                xs[u] = v < V ? load_one<2>(row, v) : -kInf;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (xs[u] < kInf && xs[u] > lm) lm = xs[u];
        }
        const float wm = wave_max(lm);
        if (l == 0) s_wkey[wave] = static_cast<int>(f32_bits(wm));
        lds_barrier();
        float mm = -kInf;
#pragma unroll
        for (int w = 0; w < 8; ++w) mm = fmaxf(mm, bits_f32(static_cast<uint32_t>(s_wkey[w])));
        return mm;
    };
    // ---- survivor records: each lane chunk whose key reaches tk (so may
    // hold x >= theta) is recorded with its first token, the wavefront's
    // records placed by ballot (no atomics) ----
    auto take_records = [&](int pb, int tk, int tkey) __attribute__((always_inline)) {
        if (!__any(tkey >= tk)) return;  // no chunk of the wavefront reaches tk
        int n = 0;
        uint4* out = s_rec[pb] + kRecCap * wave;
        int* tok_out = s_rtok[pb] + kRecCap * wave;
        uint32_t keys[4 * kGroups];
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            const uint4 kq = *reinterpret_cast<const uint4*>(&s_ck[g][tid][0]);
            keys[4 * g] = kq.x;
            keys[4 * g + 1] = kq.y;
            keys[4 * g + 2] = kq.z;
            keys[4 * g + 3] = kq.w;
        }
        // eight chunks at a time: a group is passed over unless one of its
        // keys reaches tk on some lane (the packed maximum of its keys)
        unrolled<kGroups>([&](auto gg) __attribute__((always_inline)) {
            constexpr int g = decltype(gg)::value;
            const uint32_t gm = pk_max_i16(pk_max_i16(keys[4 * g], keys[4 * g + 1]),
                                           pk_max_i16(keys[4 * g + 2], keys[4 * g + 3]));
            const int gk = max(static_cast<int>(static_cast<int16_t>(gm & 0xffffu)),
                               static_cast<int>(static_cast<int16_t>(gm >> 16)));
            if (__builtin_amdgcn_ballot_w64(gk >= tk) == 0) return;
            unrolled<8>([&](auto ii) __attribute__((always_inline)) {
                constexpr int c = 8 * g + decltype(ii)::value;
                if constexpr (c < kChunks) {
                    const int ck = static_cast<int16_t>(keys[c >> 1] >> (16 * (c & 1)));
                    const bool flagged = ck >= tk;
                    const uint64_t bal = __builtin_amdgcn_ballot_w64(flagged);
                    if (bal != 0) {
                        const int slot = n + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                                 static_cast<uint32_t>(bal >> 32),
                                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u)));
                        if (flagged && slot < kRecCap) {
                            out[slot] = make_uint4(reg[4 * c], reg[4 * c + 1], reg[4 * c + 2], reg[4 * c + 3]);
                            tok_out[slot] = 256 * (s_begin + 8 * c) + j;
                        }
                        n += __popcll(bal);
                    }
                }
            });
        });
        if (l == 0) s_nrec[pb][wave] = n;
    };

    // ---- a row's shortlist from its records, in two parts (one
    // wavefront). finish_extract, once the records are complete: the
    // survivors (positive, slot reaching tk's, so x >= theta; not statically
    // masked) into s_key and s_x, and up to 64 of them ranked in the lanes
    // (the count of survivor keys above each one's; keys are distinct).
    // finish_publish, once the row's logsumexp is known: the entries of
    // rank < M (ranked here when there were more than 64), the bound at rank
    // M (else theta), the RowInfo. More records or survivors than kept: no
    // shortlist. ----
    struct Extracted {
        int n;          // survivors, keys in s_key and values in s_x
        bool overflow;  // no shortlist
        bool in_lanes;  // n <= 64: ranked already, survivor i in lane i
        int rank;
        float x;
        uint64_t key;
        float bound_x;  // x at rank M (n > M)
    };
    auto finish_extract = [&](int pb, int tk, bool full, bool live, int bb, bool mask) __attribute__((always_inline)) {
        Extracted st;
        st.n = 0;
        st.in_lanes = false;
        st.rank = 0;
        st.x = 0.0f;
        st.key = ~0ull;
        st.bound_x = -kInf;
        // the eight wavefronts' record counts, read once
        const int4 n_lo = *reinterpret_cast<const int4*>(&s_nrec[pb][0]);
        const int4 n_hi = *reinterpret_cast<const int4*>(&s_nrec[pb][4]);
        const int nrec[8] = {n_lo.x, n_lo.y, n_lo.z, n_lo.w, n_hi.x, n_hi.y, n_hi.z, n_hi.w};
        bool overflow = full;
#pragma unroll
        for (int w = 0; w < 8; ++w) overflow = overflow || nrec[w] > kRecCap;
        if (M > 0 && live && !overflow) {
            const uint32_t thr = static_cast<uint32_t>(tk - static_cast<int>(kFixedBase - 1u));
            // the eight wavefronts' lists read as one (list w from prefix[w]),
            // 64 records a pass, one per lane
            int prefix[9];
            prefix[0] = 0;
#pragma unroll
            for (int w = 0; w < 8; ++w) prefix[w + 1] = prefix[w] + __builtin_amdgcn_readfirstlane(nrec[w]);
            const int total = prefix[8];
            const bool check = p.banned != nullptr || p.banned_pe != nullptr || mask;
            int n = 0;
#pragma unroll 1
            for (int i0 = 0; i0 < total; i0 += 64) {
                const int i = i0 + l;
                int src = 0;
#pragma unroll
                for (int w = 1; w < 8; ++w) src = i >= prefix[w] ? kRecCap * w + (i - prefix[w]) : src;
                if (i < prefix[1]) src = i;
                const bool has = i < total;
                const uint4 q = has ? s_rec[pb][src] : make_uint4(0u, 0u, 0u, 0u);
                const int t0 = has ? s_rtok[pb][src] : 0;
                const uint32_t R[4] = {q.x, q.y, q.z, q.w};
                // the record's survivors as a bit mask (element e = stripe
                // 8c + e), placed after those of the lanes below (a prefix
                // sum of the counts, bit plane by bit plane)
                uint32_t hits = 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t a = (R[e >> 1] >> (16 * (e & 1))) & 0xffffu;
                    hits |= (has && a >= thr && a < static_cast<uint32_t>(kLutHalf)) ? (1u << e) : 0u;
                }
                if (check) {
#pragma unroll 1
                    for (uint32_t h = hits; h != 0; h &= h - 1) {
                        const int e = __ffs(h) - 1;
                        if (static_masked(p, bb, t0 + 256 * e, mask)) hits &= ~(1u << e);
                    }
                }
                const int cnt = __popc(hits);
                int before = 0, pass_total = 0;
#pragma unroll
                for (int bit = 0; bit < 4; ++bit) {
                    const uint64_t plane = __ballot((cnt >> bit) & 1);
                    before += static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                  static_cast<uint32_t>(plane >> 32),
                                  __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(plane), 0u)))
                              << bit;
                    pass_total += __popcll(plane) << bit;
                }
                int slot = n + before;
#pragma unroll 1
                for (uint32_t h = hits; h != 0; h &= h - 1, ++slot) {
                    const int e = __ffs(h) - 1;
                    const uint32_t w2 = e < 4 ? (e < 2 ? R[0] : R[1]) : (e < 6 ? R[2] : R[3]);
                    const uint32_t a = (w2 >> (16 * (e & 1))) & 0xffffu;
                    if (slot < kSurvivorCap) {
                        const float x = bf16_to_f32(static_cast<uint16_t>(a + (kFixedBase - 1u)));
                        s_key[slot] = survivor_key(x, t0 + 256 * e);
                        s_x[slot] = x;
                    }
                }
                n += pass_total;
            }
            st.n = n;
            if (n > kSurvivorCap) {
                overflow = true;
            } else {
                if ((n & 1) && l == 0) s_key[n] = 0;  // a zero key pads the pairs read when ranking
                wave_sync();
                if (n <= 64) {
                    // each survivor's rank: the count of keys above its own
                    st.in_lanes = true;
                    const uint4* k2 = reinterpret_cast<const uint4*>(s_key);
                    const int npair = (n + 1) >> 1;
                    const uint64_t ki = l < n ? s_key[l] : ~0ull;
                    int rank = 0;
#pragma unroll 8
                    for (int jp = 0; jp < npair; ++jp) {
                        const uint4 a = k2[jp];
                        rank += static_cast<int>(((static_cast<uint64_t>(a.y) << 32) | a.x) > ki) +
                                static_cast<int>(((static_cast<uint64_t>(a.w) << 32) | a.z) > ki);
                    }
                    st.rank = rank;
                    st.key = ki;
                    st.x = l < n ? s_x[l] : 0.0f;
                    const uint64_t at_m = __ballot(l < n && rank == M);
                    if (at_m != 0) st.bound_x = __shfl(st.x, __ffsll(static_cast<long long>(at_m)) - 1);
                }
            }
        }
        st.overflow = overflow;
        return st;
    };
    auto finish_publish = [&](const Extracted& st, int64_t rr, float lse, float theta, bool bad) __attribute__((always_inline)) {
        const bool coherent = p.step_done != nullptr;
        RowInfo info;
        info.lse = lse;
        info.invalid = bad ? 1u : 0u;
        info.bound = -kInf;
        info.count = 0;
        const int n = st.n;
        if (M > 0 && lse != -kInf && !st.overflow) {
            ShortEntry* out = p.shortlist + rr * M;
            float bound_x = st.bound_x;
            const uint4* k2 = reinterpret_cast<const uint4*>(s_key);
            const int npair = (n + 1) >> 1;
            if (st.in_lanes && l < n && st.rank < M) {
                const int32_t tok = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(st.key & 0xffffffffu));
                publish_entry(out, st.rank, st.x - lse, tok, coherent);
            }
#pragma unroll 1
            for (int i0 = 0; !st.in_lanes && i0 < n; i0 += 64) {
                const int i = i0 + l;
                const uint64_t ki = i < n ? s_key[i] : ~0ull;
                int rank = 0;
#pragma unroll 8
                for (int jp = 0; jp < npair; ++jp) {
                    const uint4 a = k2[jp];
                    rank += static_cast<int>(((static_cast<uint64_t>(a.y) << 32) | a.x) > ki) +
                            static_cast<int>(((static_cast<uint64_t>(a.w) << 32) | a.z) > ki);
                }
                const float x = i < n ? s_x[i] : 0.0f;
                if (i < n && rank < M) {
                    const int32_t tok = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(ki & 0xffffffffu));
                    publish_entry(out, rank, x - lse, tok, coherent);
                }
                const uint64_t at_m = __ballot(i < n && rank == M);
                if (at_m != 0) bound_x = __shfl(x, __ffsll(static_cast<long long>(at_m)) - 1);
            }
            info.count = n < M ? n : M;
            const float bx = n > M ? bound_x : theta;
            info.bound = bx > -kInf ? bx - lse : -kInf;
        }
        if (M > 0 && lse != -kInf && st.overflow) info.count = -1;
        if (l == 0) publish_rowinfo(p.rowinfo + rr, info, coherent);
        signal_row_done(p, rr, l);
    };

    Extracted fin;

    // ---- the first row in flight; segment 0 arrives ----
    if (r < rows) issue_loads(r);
    if (seg == 0 && r < rows) arrive();
    // segment 0 finds each next row one step ahead, where it has time (the
    // row after the one it streams in)
    int64_t r_ahead = rows;
    int b_ahead = 0, len_ahead = 0;
    if (!tickets && seg == 0) r_ahead = next_read_row(r + gridDim.x, b_ahead, len_ahead);

    // Each routine has one static copy, which both segments run at
    // different steps (the code of a row must stay in the instruction
    // cache): phase 0, segment 1's raw maxima while wavefront kFinisher
    // finishes the previous row; the exchange and the term table (B1, B2);
    // then two steps h = 0, 1 closed by barriers B3 and B4: in step 0
    // segment 1 arrives (transposes and converts) and both record their
    // survivor chunks, and segment 0 folds its stripes; in step 1 segment
    // 0 arrives with the next row and segment 1 folds its stripes.
    while (r < rows) {
        int bn = 0, lenn = 0;
        int64_t rn = rows;
        if (tickets) {
            if (tid == kPublisher) publish_next_row(p, rows, q_next, s_rows[par ^ 1]);
        } else if (seg == 1) {
            rn = next_read_row(r + gridDim.x, bn, lenn);
        } else {
            rn = r_ahead;
            bn = b_ahead;
            lenn = len_ahead;
        }
        const bool mask_eos = new_len < min_length_of(p, b);
        const uint16_t* row = static_cast<const uint16_t*>(p.x) + r * V;

        // ---- phase 0 ----
        if (seg == 1) keys_loaded();
        const int tkey = max(static_cast<int>(static_cast<int16_t>(t_smax & 0xffffu)),
                             static_cast<int>(static_cast<int16_t>(t_smax >> 16)));
        const int tumax = static_cast<int>(max(t_umax & 0xffffu, t_umax >> 16));
        const bool tbad = tkey >= 0x7f80 || tumax > static_cast<int>(kBf16NegInf);
        const int key15 = max(tkey, 0);  // threads whose values are all negative count as +0
        if (M > 0) atomicAdd(&s_hist1[key15 >> 7], 1);
        const int wkey = wave_max_int(tkey);
        const bool wbad = __any(tbad);
        if (l == 0) {
            s_wkey[wave] = wkey;
            s_wbad[wave] = wbad ? 1 : 0;
        }
        lds_barrier();
        int mkey = -32768;
        bool any_bad = false;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            mkey = max(mkey, s_wkey[w]);
            any_bad = any_bad || s_wbad[w] != 0;
        }
        float m = mkey >= 0 ? pattern_value<2>(static_cast<uint32_t>(mkey)) : -kInf;
        // a NaN or +inf, or every value negative: the maximum comes from memory
        const bool need_m = any_bad || mkey < 0;
        const bool fast = !need_m && table_fits_fixed(m);
        const bool select = M > 0 && !any_bad;
        int b1 = 0, above1 = 0;
        if (select) {
            hist_select(s_hist1, M, l, b1, above1);
            if ((key15 >> 7) == b1) atomicAdd(&s_hist2[key15 & 127], 1);
        }
        if (fast) {
            // the 8192 slots, 16 per thread (slots tid + 512 i, the negative
            // half from i = 8): slot 0 exp(-m), slot k magnitude base - 1 + k;
            // positive slots above m hold 0
            const uint32_t mp = f32_bits(m) >> 16;
            const float em = exp_nonpositive(-m);
#pragma unroll 4
            for (int i = 0; i < 2 * kLutHalf / kRlThreads; ++i) {
                const bool neg = i >= kLutHalf / kRlThreads;
                const int k = tid + kRlThreads * (i % (kLutHalf / kRlThreads));
                const uint32_t u = kFixedBase - 1u + static_cast<uint32_t>(k);
                const bool valid = neg || u <= mp;
                const float x = bf16_to_f32(static_cast<uint16_t>((neg ? 0x8000u : 0u) | u));
                const float t = exp_nonpositive_nb(x - m);
                lut[(neg ? kLutHalf : 0) + k] = k == 0 ? em : (valid ? t : 0.0f);
            }
        }
        lds_barrier();
        if (tid < 256) s_hist1[tid] = 0;  // every wavefront has its b1
        // theta: the M-th largest thread maximum (M values reach it), raised
        // to 2^-25 where that is smaller (fewer than M values are above it;
        // then every value from 2^-25 up is a survivor and every value left
        // out is below theta): theta is a pattern the table slots keep
        int tk = static_cast<int>(kFixedBase);
        if (select) {
            int b2 = 0, above2 = 0;
            hist_select(s_hist2, M - above1, l, b2, above2);
            tk = max((b1 << 7) | b2, static_cast<int>(kFixedBase));
        }
        const float theta = M > 0 ? (select ? pattern_value<2>(static_cast<uint32_t>(tk)) : -kInf) : kInf;
        // the shortlist comes from records of table slots: rows on the
        // table path; others keep none (the select pass reads the row)
        const bool records = select && fast;
        const bool full = M > 0 && !records;
        if (need_m) m = memory_max(row);
        const bool do_lse = m > -kInf;

        // ---- phases A and B. A row the table does not cover runs the
        // chain for its loads only and folds from memory. ----
        if (tickets) {
            int bt = 0, lt = 0;
            rn = read_row_slot(s_rows[par ^ 1], bt, lt);  // published before the first barrier
            bn = bt;
            lenn = lt;
        }
#pragma unroll 1
        for (int h = 0; h < 2; ++h) {
            if ((h == 0) == (seg == 1) && (h == 0 || rn < rows)) arrive();
            // the row's records are complete (B3): its survivors
            if (h == 1 && wave == kFinisher) fin = finish_extract(par, tk, full, do_lse, b, mask_eos);
            if (h == 1 && seg == 0 && !tickets && rn < rows) r_ahead = next_read_row(rn + gridDim.x, b_ahead, len_ahead);
            if (h == 0 && records) {
                const int tk_thread = max(static_cast<int>(static_cast<int16_t>(t_smax & 0xffffu)),
                                          static_cast<int>(static_cast<int16_t>(t_smax >> 16)));
                take_records(par, tk, tk_thread);
            }
            if ((h == 0) == (seg == 0)) {
                const float a0 = seg == 0 ? 0.0f : s_acc[par][j];
                float acc = chain_table(a0, rn);
                if (!fast) acc = do_lse ? chain_memory(a0, m, row) : a0;
                s_acc[par][j] = acc;
            }
            lds_barrier();  // h = 0: B3, h = 1: B4
            if (h == 0 && seg == 0) s_hist2[tid] = 0;  // every wavefront has its b2
        }
        // ---- the row's end (phase 0 of the next row): its lane tree,
        // logsumexp, ranked shortlist and RowInfo ----
        if (wave == kFinisher) {
            float lse = -kInf;
            if (do_lse) {
                float a[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) a[e] = s_acc[par][4 * l + e];
                lse = logsumexp_from(m, lane_tree_sum(a, l));
            }
            finish_publish(fin, r, lse, theta, any_bad);
            if (l < 8) s_nrec[par][l] = 0;
        }

        r = rn;
        b = bn;
        new_len = lenn;
        par ^= 1;
    }
}

int g_relay_cus[64];

}  // namespace

// bfloat16 logits rows of at most 155648 entries, V % 8 == 0, 16-byte
// aligned, shortlists of at most 256 entries.
bool row_relay_eligible(const DecodeParams& p) {
    if (p.dtype != 2 || !p.from_logits) return false;
    if (p.V % 8 != 0 || reinterpret_cast<uintptr_t>(p.x) % 16 != 0) return false;
    if ((p.V + 255) / 256 > kRlStripes) return false;
    return p.M <= 256;
}

bool row_relay_preferred(const DecodeParams& p) { return (p.V + 255) / 256 >= (3 * kRlStripes) / 4; }

hipError_t launch_row_relay(const DecodeParams& p, int64_t rows, hipStream_t stream) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    if (g_relay_cus[device] == 0) {
        int cus = 0;
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
        if (e != hipSuccess) return e;
        g_relay_cus[device] = cus > 0 ? cus : 1;
    }
    // one workgroup per CU, less the CUs left to an overlapped select pass
    const int64_t cus = g_relay_cus[device] - p.reserve_cus > 0 ? g_relay_cus[device] - p.reserve_cus : 1;
    const int64_t grid = rows < cus ? rows : cus;
    // the first chunk that may reach past the row on some lane: segment 0
    // ends at stripe per (or the row), segment 1 at the row's end; wavefront
    // 3's lane 63 starts a chunk's 16-byte groups last
    const int S = (p.V + 255) / 256;
    const int per = ((((S + 1) / 2) + 7) / 8) * 8;
    int first_partial = kRlChunks;
    for (int sg = 0; sg < 2; ++sg) {
        const int end_r = p.V < 256 * (sg * per + per) ? p.V : 256 * (sg * per + per);
        const int c_all = (end_r - (256 * (sg * per + 7) + 64 * 3 + 56) + 2047) >> 11;
        first_partial = c_all < first_partial ? c_all : first_partial;
    }
    // segments of at most 256 stripes (V <= 131072) fit 32 chunks: the
    // chunks past them would only add +0 terms
    const dim3 g(static_cast<unsigned>(grid)), blk(kRlThreads);
    if (per <= 8 * kRlChunksShort) {
        if (first_partial >= kRlChunksShort - 4)
            hipLaunchKernelGGL((row_relay_kernel<kRlChunksShort, kRlChunksShort - 4>), g, blk, 0, stream, p, rows);
        else
            hipLaunchKernelGGL((row_relay_kernel<kRlChunksShort, 0>), g, blk, 0, stream, p, rows);
    } else if (first_partial >= kRlChunks - 4) {
        hipLaunchKernelGGL((row_relay_kernel<kRlChunks, kRlChunks - 4>), g, blk, 0, stream, p, rows);
    } else {
        hipLaunchKernelGGL((row_relay_kernel<kRlChunks, 0>), g, blk, 0, stream, p, rows);
    }
    return hipGetLastError();
}

}  // namespace dbs_hip
