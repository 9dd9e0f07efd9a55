// SPDX-License-Identifier: MIT
//
// Row pass for bfloat16 logits rows that keeps HBM streaming while rows are
// worked on.
//
// The logsumexp of the reference folds exp(x - max) into 256 lanes (lane j =
// v mod 256, increasing v; reference src/kernels_scalar.cpp:48-66): each
// lane's sum is one sequential chain, and the row maximum is needed before
// its first term. Here one workgroup of 256 threads per CU (one wavefront
// per SIMD) is persistent over rows, and thread j owns fold lane j of the
// whole row: its 8 * NCH stripes (stripe s = elements 256 s .. 256 s + 255)
// sit in 4 * NCH registers, two stripes per register, so every wavefront's
// chains run at once and independently.
//
// Data path: each wavefront streams its 1 KB chunks (8 stripes x its 64
// lanes) from HBM with 16-byte buffer loads into registers, kD chunks ahead
// of their use, so kD KB per wavefront stay in flight across every per-row
// phase. A chunk is transposed through a 1 KB LDS slot of the wavefront (one
// 16-byte write per lane, two transposing reads) into the registers it
// belongs to, as soon as the chain of the row before has read them. (Loads
// into registers, not LDS-DMA: the waits on the vector memory counter are
// exact for the former, while an LDS-DMA load has been seen not to have
// landed in LDS at a wait that counts it complete.)
//
// Per row, between two chains: the row maximum, NaN/+inf flag and a
// shortlist threshold (the min over the wavefronts of each wavefront's
// ceil(M/4)-th largest thread maximum: at least M elements reach it) are
// exchanged through LDS; wavefront 0 finishes the previous row (fixed lane
// tree, logsumexp, shortlist by rank, RowInfo) while the others build the
// row's table of exact terms exp(fl(x - m)) by bfloat16 pattern. During the
// chain, elements reaching the threshold are recorded (from the registers)
// for the shortlist. Rows the table does not cover fold with the Cephes
// evaluation from the registers.
#include <hip/hip_runtime.h>

#include <utility>

#include "row_helpers.hpp"

namespace dbs_hip {

namespace {

constexpr int kStThreads = 256;  // four wavefronts, fold lane = thread
// Chunk loads in flight per wavefront: 16, or 15 where that divides the
// chunk count (chunk c of every row uses load slot c % kD).
template <int NCH>
constexpr int loads_in_flight() {
    return NCH % 16 == 0 ? 16 : NCH % 15 == 0 ? 15 : NCH % 14 == 0 ? 14 : NCH % 13 == 0 ? 13 : 12;
}
constexpr uint32_t kBf16NegInf = 0xff80u;
constexpr int kBf16PosInf = 0x7f80;

typedef __attribute__((address_space(3))) unsigned char st_lds_u8;

// f(integral_constant<int, i>) for i = 0 .. N - 1, expanded at compile time
// (the chunk loops index the register array with constants only, whatever
// the unroller would decide for bodies this large).
template <class F, int... I>
__device__ __forceinline__ void static_for_seq(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// A chunk through the wavefront's LDS slot: lane L writes its 16 bytes at
// byte 16 L, then reads 8 bytes at 128 (a / 4) + 32 G + 8 (a % 4) and at
// +512 (L = 16 G + a) transposed (see the chunk layout below). LDS operations
// of one wavefront take effect in order: no wait between the write and the
// reads, nor before the next chunk's write. The values are tied to the wait
// for the reads (slot_wait).
__device__ __forceinline__ void slot_pass(uint32_t waddr, uint32_t raddr, const v4u32& q, v2u32& lo, v2u32& hi) {
    asm volatile(
        "ds_write_b128 %2, %3\n\t"
        "ds_read_b64_tr_b16 %0, %4\n\t"
        "ds_read_b64_tr_b16 %1, %4 offset:512"
        : "=&v"(lo), "=&v"(hi)
        : "v"(waddr), "a"(q), "v"(raddr)
        : "memory");
}

// A chunk's 16-byte load into AGPRs (where it stays until its slot pass).
// Inline assembly, so that the compiler neither waits for it nor moves its
// registers while it is in flight; chunk_wait waits for it.
__device__ __forceinline__ void chunk_load(v4u32& dst, const v4u32& rsrc, int voffset) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=a"(dst) : "v"(voffset), "s"(rsrc) : "memory");
}

// Buffer descriptor of bytes [0, nbytes) at p (loads past the end read 0),
// in scalar registers.
__device__ __forceinline__ v4u32 buffer_desc(const void* p, int nbytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    v4u32 d;
    d.x = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
    d.y = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32)) & 0xffffu;
    d.z = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(nbytes));
    d.w = 0x00020000u;
    return d;
}

// The oldest chunk load of the wavefront has arrived once at most kD - 1
// vector memory operations are outstanding (loads into registers complete in
// order; any other operation counted was issued after it, or completes before
// it is counted out).
template <int kD>
__device__ __forceinline__ void chunk_wait(v4u32& q) {
    asm volatile("s_waitcnt vmcnt(%1)" : "+a"(q) : "n"(kD - 1) : "memory");
}

// Waits until at most N LDS operations of this wavefront are outstanding;
// the slot's values are ready after it (ties them to the wait).
template <int N>
__device__ __forceinline__ void slot_wait(v2u32& lo, v2u32& hi) {
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(lo), "+v"(hi) : "n"(N) : "memory");
}

// The k-th largest (1-based, 1 <= k <= 256) of the workgroup's 256 keys in
// [0, 32767] (four per lane of the calling wavefront, in keys), by a bitwise
// search over ballots. Every lane gets it.
__device__ __forceinline__ int block_kth_largest(const int4& keys, int k) {
    uint32_t prefix = 0;
    for (int bit = 14; bit >= 0; --bit) {
        const int cand = static_cast<int>(prefix | (1u << bit));
        const int n = __popcll(__ballot(keys.x >= cand)) + __popcll(__ballot(keys.y >= cand)) +
                      __popcll(__ballot(keys.z >= cand)) + __popcll(__ballot(keys.w >= cand));
        if (n >= k) prefix = static_cast<uint32_t>(cand);
    }
    return static_cast<int>(prefix);
}

constexpr int kRecCap = 64;  // survivor records kept per wavefront and row

// The k-th largest (1-based) survivor candidates of a row, from its records:
// record i of wavefront w holds one lane's chunk (eight bfloat16 values,
// tokens tok[i] + 256 e, e = 0..7) that reached the threshold somewhere.
// One wavefront turns them into survivors (finite x >= theta, not statically
// masked: banned, EOS below min_length), places each by its rank (the count
// of survivor keys above its own; keys are distinct), writes the shortlist
// (log-probs x - lse) and, at rank M, the bound on the tokens left out (else
// theta), then the RowInfo and the row's count for the overlapped decode.
// More records or survivors than kept: no shortlist.
__device__ void finish_row_lean(const DecodeParams& p, int64_t r, float lse, float theta, const uint4* rec,
                                const int* rec_tok, const int (&nrec)[4], uint64_t* s_key, float* s_x, int lane,
                                int b, bool mask_eos) {
    const int M = p.M;
    const bool coherent = p.step_done != nullptr;
    RowInfo info;
    info.lse = lse;
    info.invalid = 0u;
    info.bound = -kInf;
    info.count = 0;
    bool overflow = nrec[0] > kRecCap || nrec[1] > kRecCap || nrec[2] > kRecCap || nrec[3] > kRecCap;
    if (M > 0 && lse != -kInf && !overflow) {
        // records -> survivor list (one record per lane, eight values each)
        int n = 0;
#pragma unroll 1
        for (int w = 0; w < 4; ++w) {
#pragma unroll 1
            for (int i0 = 0; i0 < nrec[w]; i0 += 64) {
                const int i = i0 + lane;
                uint4 q = make_uint4(0u, 0u, 0u, 0u);
                int t0 = 0;
                if (i < nrec[w]) {
                    q = rec[kRecCap * w + i];
                    t0 = rec_tok[kRecCap * w + i];
                }
                const uint32_t R[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float x = bf16_to_f32(static_cast<uint16_t>(R[e / 2] >> (16 * (e & 1))));
                    const int v = t0 + 256 * e;
                    const bool hit = i < nrec[w] && x >= theta && x < kInf && !static_masked(p, b, v, mask_eos);
                    const uint64_t bal = __ballot(hit);
                    const int slot = n + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                             static_cast<uint32_t>(bal >> 32),
                                             __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u)));
                    if (hit && slot < kSurvivorCap) {
                        s_key[slot] = survivor_key(x, v);
                        s_x[slot] = x;
                    }
                    n += __popcll(bal);
                }
            }
        }
        if (n > kSurvivorCap) {
            overflow = true;
        } else {
            if ((n & 1) && lane == 0) s_key[n] = 0;  // a zero key pads the pairs read below
            wave_sync();
            ShortEntry* out = p.shortlist + r * M;
            const uint4* k2 = reinterpret_cast<const uint4*>(s_key);
            const int npair = (n + 1) >> 1;
            float bound_x = -kInf;
#pragma unroll 1
            for (int i0 = 0; i0 < n; i0 += 64) {
                const int i = i0 + lane;
                const uint64_t ki = i < n ? s_key[i] : ~0ull;
                int rank = 0;
#pragma unroll 1
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
    }
    if (M > 0 && lse != -kInf && overflow) info.count = -1;
    if (lane == 0) publish_rowinfo(p.rowinfo + r, info, coherent);
    signal_row_done(p, r, lane);
}

struct RowState {
    int64_t r;
    int b, len;
    float m;
    float theta;
    int tk1;  // a chunk is looked at for survivors when its largest signed pattern reaches this
    int ulo;  // table base (see table_fits)
    bool valid, fast, mask_eos;
};

// Rows by the workgroup's fixed stride over the processing order (which is
// step-major in the overlapped decode), never by tickets: every row costs the
// same here, and a ticket's atomic would be waited for (with the loads in
// flight) where its result is moved.
template <int NCH>
__global__ __launch_bounds__(kStThreads, 1) void row_stream_kernel(DecodeParams p, int64_t rows) {
    constexpr int NREG = 4 * NCH;
    constexpr int kD = loads_in_flight<NCH>();
    static_assert(NCH % kD == 0, "chunk c of every row uses load slot c % kD");
    constexpr int kMinPartial = 32;   // V > 65536: chunks below this one are full
    // (the table first, at LDS address 0: its lookups need no base added)
    __shared__ __attribute__((aligned(1024))) float lut[2 * kLutHalf];
    __shared__ __attribute__((aligned(16))) unsigned char stage[4 * 1024];
    __shared__ __attribute__((aligned(16))) int16_t s_ck[NCH * kStThreads];
    __shared__ float s_acc[kStThreads];
    __shared__ __attribute__((aligned(16))) uint4 s_rec[4 * kRecCap];
    __shared__ int s_tok[4 * kRecCap];
    __shared__ __attribute__((aligned(16))) uint64_t s_key[kSurvivorCap + 2];
    __shared__ float s_x[kSurvivorCap];
    __shared__ int s_ex[2][4][4];
    __shared__ __attribute__((aligned(16))) int s_tkey[kStThreads];
    __shared__ int s_tk[2];
    __shared__ RowSlot s_rows[4];

    const int tid = static_cast<int>(threadIdx.x);
    const int l = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int V = p.V, M = p.M;

    // Chunk c of wavefront w: stripes 8c .. 8c + 7, lanes 64 w .. 64 w + 63.
    // Lane L's 16-byte load brings stripe 8c + L / 8, lanes 64 w + 8 (L % 8)
    // .. + 7 (bytes 4096 c + 512 (L / 8) + 128 w + 16 (L % 8) of the row),
    // written to byte 16 L of the slot, i.e. (stripe i, lane n) at byte
    // 128 i + 2 n.
    const uint32_t wslot = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(stage + w * 1024));
    const uint32_t wr0 = wslot + 16 * l;
    const uint32_t rd0 = wslot + 128 * ((l & 15) >> 2) + 32 * (l >> 4) + 8 * (l & 3);
    const int voff = 512 * (l >> 3) + 128 * w + 16 * (l & 7);
    auto view = [&](int64_t rr) {
        const bool any = rr < rows;
        const uint16_t* base = static_cast<const uint16_t*>(p.x) + (any ? rr : 0) * static_cast<int64_t>(V);
        return buffer_desc(base, any ? 2 * V : 0);
    };
    // the loads in flight: chunk j's into inflight[j % kD]
    v4u32 inflight[kD];
    int voffr = voff;  // (per-row opaque copy: the chunk offsets are added per chunk, not kept)
    auto load = [&](const v4u32& rs, int slot, int c) __attribute__((always_inline)) {
        // the chunk's offset in the vector offset, so that the buffer's range
        // check covers it (bytes past the row read as 0)
        chunk_load(inflight[slot], rs, voffr + 4096 * c);
    };

    // Thread j's fold lane: register 4c + q holds stripes 8c + 2q (low half)
    // and 8c + 2q + 1 (high half), i.e. tokens 256 (8c + 2q) + j and
    // 256 (8c + 2q + 1) + j. (More than the 256 VGPRs of a lane: the compiler
    // keeps part of them in AGPRs.)
    uint32_t reg[NREG];
    // Per chunk and thread, the largest signed 16-bit pattern over its eight
    // values (the largest value wherever one is non-negative), in s_ck: the
    // chain reads chunk c's of the row it folds before the next row's chunk
    // c replaces it. And the running packed signed and unsigned pattern
    // maxima of the incoming row (the row maximum where it is >= +0; +inf and
    // NaN of either sign).
    uint32_t t_smax = 0x80008000u, t_umax = 0u;
    // (Vr, jr: per-row opaque copies of V and the lane, so that nothing the
    // unrolled chunks derive from them is hoisted out of the row loop into
    // registers)
    int Vr = V, jr = tid;
    auto place = [&](auto cc, const v2u32& lo, const v2u32& hi) __attribute__((always_inline)) {
        constexpr int c = decltype(cc)::value;
        uint32_t R[4] = {lo.x, lo.y, hi.x, hi.y};
        if constexpr (c >= kMinPartial) {
            if (2048 * (c + 1) > Vr) {  // elements past the row become -inf
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const bool lo_out = 256 * (8 * c + 2 * q) + jr >= Vr;
                    const bool hi_out = 256 * (8 * c + 2 * q + 1) + jr >= Vr;
                    R[q] = (lo_out ? kBf16NegInf : (R[q] & 0xffffu)) |
                           (hi_out ? (kBf16NegInf << 16) : (R[q] & 0xffff0000u));
                }
            }
        }
        const uint32_t kc = pk_max_i16(pk_max_i16(R[0], R[1]), pk_max_i16(R[2], R[3]));
        t_smax = pk_max_i16(t_smax, kc);
        t_umax = pk_max_u16(pk_max_u16(t_umax, pk_max_u16(R[0], R[1])), pk_max_u16(R[2], R[3]));
#pragma unroll
        for (int q = 0; q < 4; ++q) reg[4 * c + q] = R[q];
        const uint32_t ck = static_cast<uint32_t>(max(static_cast<int>(static_cast<int16_t>(kc & 0xffffu)),
                                                      static_cast<int>(static_cast<int16_t>(kc >> 16)))) & 0xffffu;
        s_ck[kStThreads * c + tid] = static_cast<int16_t>(ck);
        // computed here, while the chunk is in VGPRs, not sunk past the chain
        asm volatile("" : "+v"(t_smax), "+v"(t_umax));
    };

    // ---- the workgroup's rows, published by thread 0 three ahead ----
    int64_t q_next = 0, q_pre = 0;  // thread 0: processing index, and the next one fetched ahead
    if (tid == 0) {
        q_next = first_ticket<false>(p);
        int b0 = 0, len0 = 0;
        s_rows[0].r = find_read_row<false>(p, rows, q_next, b0, len0);
        s_rows[0].b = b0;
        s_rows[0].len = len0;
        publish_next_row<false>(p, rows, q_next, s_rows[1]);
        publish_next_row<false>(p, rows, q_next, s_rows[2]);
    }
    lds_barrier();
    auto row_at = [&](int k, int& b, int& len) { return read_row_slot(s_rows[k & 3], b, len); };

    // ---- prologue: row 0 into the registers ----
    {
        int bt = 0, lt = 0;
        const v4u32 rs0 = view(row_at(0, bt, lt)), rs1 = view(row_at(1, bt, lt));
        asm volatile("" : "+v"(voffr));
        static_for<kD>([&](auto cc) __attribute__((always_inline)) {
            load(rs0, decltype(cc)::value, decltype(cc)::value);
        });
        // the index for the first row boundary
        if (tid == 0) q_pre = q_next < rows ? next_index<false>(p, q_next) : rows;
        asm volatile("" : "+s"(Vr));
        asm volatile("" : "+v"(jr));
        static_for<NCH>([&](auto cc) __attribute__((always_inline)) {
            constexpr int c = decltype(cc)::value;
            v2u32 lo, hi;
            chunk_wait<kD>(inflight[c % kD]);
            slot_pass(wr0, rd0, inflight[c % kD], lo, hi);
            slot_wait<0>(lo, hi);
            place(cc, lo, hi);
            if constexpr (c + kD < NCH) load(rs0, c % kD, c + kD);
            else load(rs1, c % kD, c + kD - NCH);
        });
    }

    int k = 0;  // index of the current row
    RowState pend{};
    pend.valid = false;
    int wrec = 0;  // survivor records the wavefront wrote for the row just folded

    // The phase between two chains: the incoming row k's statistics, the
    // previous row's finish and row k's threshold (wavefront 0) and row k's
    // table (the others). Rows the table cannot take (NaN/+inf, maximum below
    // 1 or -inf) are left to the fixup kernel.
    auto between_rows = [&]() {
        RowState nx{};
        nx.r = row_at(k, nx.b, nx.len);
        nx.valid = nx.r < rows;
        // the thread's largest signed pattern: its maximum where that is
        // >= +0 (negative: every value of the thread is negative)
        const int tkey = max(static_cast<int>(static_cast<int16_t>(t_smax & 0xffffu)),
                             static_cast<int>(static_cast<int16_t>(t_smax >> 16)));
        const int tumax = static_cast<int>(max(t_umax & 0xffffu, t_umax >> 16));
        const bool tbad = tkey >= kBf16PosInf || tumax > static_cast<int>(kBf16NegInf);
        int wkey = tkey, wumax = tumax;
        for (int off = 32; off > 0; off >>= 1) {
            wkey = max(wkey, __shfl_xor(wkey, off));
            wumax = max(wumax, __shfl_xor(wumax, off));
        }
        const bool wbad = __any(tbad);
        const int ph = k & 1;
        s_tkey[tid] = tkey > 0 ? tkey : 0;
        if (l == 0) {
            s_ex[ph][w][0] = wkey;
            s_ex[ph][w][1] = wbad ? 1 : 0;
            s_ex[ph][w][2] = wumax;
            s_ex[ph][w][3] = wrec;
        }
        if (tid == 0) {
            // row k + 3 from the processing index fetched during the chain
            // (its atomic completed long ago: no wait on the loads in flight)
            int b3 = 0, len3 = 0;
            int64_t r3 = rows;
            if (q_next < rows) {
                q_next = q_pre;
                r3 = find_read_row<false>(p, rows, q_next, b3, len3);
            }
            s_rows[(k + 3) & 3].r = r3;
            s_rows[(k + 3) & 3].b = b3;
            s_rows[(k + 3) & 3].len = len3;
        }
        lds_barrier();
        int mkey = -32768, umax = 0;
        bool any_bad = false;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            mkey = max(mkey, s_ex[ph][ww][0]);
            any_bad = any_bad || s_ex[ph][ww][1] != 0;
            umax = max(umax, s_ex[ph][ww][2]);
        }
        // a negative largest pattern: every value is negative (below 1)
        const float m = mkey >= 0 ? pattern_value<2>(static_cast<uint32_t>(mkey)) : -1.0f;
        nx.m = m;
        nx.fast = nx.valid && !any_bad && table_fits(m, nx.ulo);
        nx.mask_eos = nx.valid && nx.len < min_length_of(p, nx.b);
        t_smax = 0x80008000u;
        t_umax = 0u;
        if (tid == 0 && nx.valid && !nx.fast) {
            const unsigned long long i = atomicAdd(p.fixup_count, 1ull);
            p.fixup_rows[i] = nx.r;
        }

        if (w == 0) {
            // row k's threshold: the M-th largest thread maximum (M threads
            // reach it, so M values do), or, where fewer than M threads hold
            // a value > +0, the smallest positive value (every positive value
            // is then a survivor, fewer than M of them maybe; every value
            // left out is <= +0, below theta)
            if (M > 0 && nx.fast) {
                const int4 keys = *reinterpret_cast<const int4*>(s_tkey + 4 * l);
                const int tk = max(block_kth_largest(keys, M), 1);
                if (l == 0) s_tk[ph] = tk;
            }
            if (pend.valid) {
                // finish the previous row: lane tree, logsumexp, shortlist
                float a4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) a4[e] = s_acc[4 * l + e];
                uint64_t zero = 0;  // per-row opaque zero: the log's constants are not hoisted
                asm volatile("" : "+s"(zero));
                const float lse = logsumexp_from_opaque(pend.m, lane_tree_sum(a4, l), zero);
                int nrec[4];
#pragma unroll
                for (int ww = 0; ww < 4; ++ww)
                    nrec[ww] = __builtin_amdgcn_readfirstlane(s_ex[ph][ww][3]);
                finish_row_lean(p, pend.r, lse, pend.theta, s_rec, s_tok, nrec, s_key, s_x, l, pend.b,
                                pend.mask_eos);
            }
        } else if (nx.fast) {
            // the table of exact terms for row k (wavefronts 1-3): slot 0
            // exp(-m), slot i >= 1 magnitude u_lo - 1 + i, per sign, as far
            // as the row's values reach (the positive ones up to m, the
            // negative ones up to the largest negative magnitude; the slot
            // for clamped magnitudes, 4095, holds 0)
            const uint32_t mp = f32_bits(m) >> 16;
            const int npos = min(kLutHalf, static_cast<int>(mp) - (nx.ulo - 1) + 1);
            const int nneg = umax >= 0x8000 ? min(kLutHalf, (umax & 0x7fff) - (nx.ulo - 1) + 1) : 1;
            const int nall = npos + max(nneg, 1);
            const float em = exp_nonpositive(-m);
#pragma unroll 1
            for (int e = tid - 64; e < nall; e += kStThreads - 64) {
                const bool neg = e >= npos;
                const int kk = neg ? e - npos : e;
                const int u = nx.ulo - 1 + kk;
                const bool ok = u < 0x7f80;
                const float xv = bf16_to_f32(static_cast<uint16_t>((neg ? 0x8000 : 0) | (ok ? u : 0)));
                const float t = exp_nonpositive_nb(xv - m);
                lut[(neg ? kLutHalf : 0) + kk] = kk == 0 ? em : (ok ? t : 0.0f);
            }
        }
        lds_barrier();
        // row k's threshold, from wavefront 0 (theta > +0): a chunk can hold
        // a value reaching it only where its largest signed pattern reaches
        // theta's
        const int tk = (M > 0 && nx.fast) ? s_tk[ph] : 0;
        nx.theta = tk > 0 ? pattern_value<2>(static_cast<uint32_t>(tk)) : kInf;
        nx.tk1 = tk > 0 ? tk : 32768;
        return nx;
    };

    RowState cur = between_rows();
    int bt = 0, lt = 0;
    while (cur.valid) {
        const v4u32 rs_n = view(row_at(k + 1, bt, lt)), rs_nn = view(row_at(k + 2, bt, lt));
        // the processing index for the next row boundary, fetched now: its
        // atomic completes during the chain, so reading it there waits on no
        // load in flight
        if (tid == 0) q_pre = q_next < rows ? next_index<false>(p, q_next) : rows;
        asm volatile("" : "+s"(Vr));
        asm volatile("" : "+v"(jr));
        asm volatile("" : "+v"(voffr));
        // ---- the chain of row k; row k + 1 comes into the registers ----
        // (every row runs it; a row left to the fixup kernel folds terms of
        // whatever table is there and keeps nothing)
        float acc = 0.0f;
        const int tk1 = cur.tk1;
        uint4* wrec_out = s_rec + kRecCap * w;
        int* wtok_out = s_tok + kRecCap * w;
        wrec = 0;
        // table index of a pattern: magnitude - (u_lo - 1) saturated at 0
        // (slot 0) and clamped to 4095, plus 4096 for negative x
        const uint32_t base2 = static_cast<uint32_t>(cur.ulo - 1) * 0x10001u;
        auto lookup = [&](auto cc, int q, float& lo, float& hi) __attribute__((always_inline)) {
            const uint32_t R = reg[4 * decltype(cc)::value + q];
            uint32_t idx = pk_sub_sat_u16(R & 0x7fff7fffu, base2);
            idx = pk_min_u16(idx, 0x0fff0fffu);
            idx |= (R >> 3) & 0x10001000u;
            const uint32_t addr = pk_shl2_u16(idx);
            lo = lut[(addr & 0xffffu) >> 2];
            hi = lut[addr >> 18];
        };
        // chunk 0 of row k + 1 through the slot (each chunk's transpose is
        // issued a chunk ahead of its placing)
        v2u32 lo_c, hi_c, lo_n, hi_n;
        chunk_wait<kD>(inflight[0]);
        slot_pass(wr0, rd0, inflight[0], lo_c, hi_c);
        float now[8], nxt[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) lookup(std::integral_constant<int, 0>{}, q, now[2 * q], now[2 * q + 1]);
        int ck_now = s_ck[tid], ck_nxt = 0;  // chunk c's key of row k (read a chunk ahead)
        static_for<NCH>([&](auto cc) __attribute__((always_inline)) {
            constexpr int c = decltype(cc)::value;
            __builtin_amdgcn_sched_barrier(0);
            // a lane whose chunk c may hold a survivor records the chunk,
            // before its registers take row k + 1
            const bool cand = ck_now >= tk1;
            if (__any(cand)) {
                const uint64_t bal = __ballot(cand);
                const int slot = wrec + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                            static_cast<uint32_t>(bal >> 32),
                                            __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u)));
                if (cand && slot < kRecCap) {
                    wrec_out[slot] = make_uint4(reg[4 * c], reg[4 * c + 1], reg[4 * c + 2], reg[4 * c + 3]);
                    wtok_out[slot] = 2048 * c + jr;
                }
                wrec += __popcll(bal);
            }
            __builtin_amdgcn_sched_barrier(0);
            // the load kD chunks on, into the slot chunk c's data left (its
            // transpose was issued a chunk ago); then chunk c + 1's transpose
            if constexpr (c + kD < NCH) load(rs_n, c % kD, c + kD);
            else load(rs_nn, c % kD, c + kD - NCH);
            if constexpr (c + 1 < NCH) {
                chunk_wait<kD>(inflight[(c + 1) % kD]);
                slot_pass(wr0, rd0, inflight[(c + 1) % kD], lo_n, hi_n);
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (c + 1 < NCH) {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    lookup(std::integral_constant<int, c + 1>{}, q, nxt[2 * q], nxt[2 * q + 1]);
                ck_nxt = s_ck[kStThreads * (c + 1) + tid];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < 8; ++q) acc = acc + now[q];
            asm volatile("" : "+v"(acc));  // the terms are added here, not sunk past the chunks after
            __builtin_amdgcn_sched_barrier(0);
            // row k + 1's chunk c into the registers: at least 15 LDS
            // operations were issued after its transposing reads, except at
            // the last chunk
            if constexpr (c + 1 < NCH) slot_wait<15>(lo_c, hi_c);
            else slot_wait<0>(lo_c, hi_c);
            place(cc, lo_c, hi_c);
#pragma unroll
            for (int q = 0; q < 8; ++q) now[q] = nxt[q];
            ck_now = ck_nxt;
            lo_c = lo_n;
            hi_c = hi_n;
        });
        s_acc[tid] = acc;
        pend = cur;
        pend.valid = cur.fast;
        ++k;
        cur = between_rows();
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load outlives the workgroup
}

int g_stream_cus[64];

template <int NCH>
hipError_t launch_stream(const DecodeParams& p, int64_t rows, int device, hipStream_t stream) {
    const int64_t cus = g_stream_cus[device] - p.reserve_cus > 0 ? g_stream_cus[device] - p.reserve_cus : 1;
    const int64_t grid = rows < cus ? rows : cus;
    hipLaunchKernelGGL((row_stream_kernel<NCH>), dim3(static_cast<unsigned>(grid)), dim3(kStThreads), 0, stream, p,
                       rows);
    return hipGetLastError();
}

}  // namespace

// bfloat16 logits rows of 65537 to 153600 entries, V % 8 == 0, 16-byte
// aligned (smaller rows keep the resident kernel).
bool row_stream_eligible(const DecodeParams& p) {
    if (p.dtype != 2 || !p.from_logits) return false;
    if (p.V % 8 != 0 || reinterpret_cast<uintptr_t>(p.x) % 16 != 0) return false;
    return p.V > 65536 && p.V <= 75 * 2048 && p.M <= 256;
}

hipError_t launch_row_stream(const DecodeParams& p, int64_t rows, hipStream_t stream) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    if (g_stream_cus[device] == 0) {
        int cus = 0;
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
        if (e != hipSuccess) return e;
        g_stream_cus[device] = cus > 0 ? cus : 1;
    }
    if (p.V <= 64 * 2048) return launch_stream<64>(p, rows, device, stream);
    return launch_stream<75>(p, rows, device, stream);
}

}  // namespace dbs_hip
