// SPDX-License-Identifier: MIT
//
// One-read row pass for decodes that take log-probabilities (not logits).
//
// Such a row has no logsumexp to fold (reference src/decoder.cpp:122-187
// reads the log-prob itself); the row pass only flags NaN / +inf and keeps
// the shortlist: the best M allowed tokens by (log-prob desc, token asc) and
// an upper bound on every allowed token left out (the row scan of reference
// src/kernels.hpp:54-140, src/kernels_scalar.cpp:16-79, restated as a
// threshold and a survivor list). Both need the row twice — the threshold
// from the whole row, then the survivors above it — so the row stays in
// VGPRs in between and is read from HBM once:
//
//   * one 256-thread workgroup per row; the row is cut into 16-byte blocks
//     aligned in memory (the first may start before the row, the last end
//     after it; a block holding a row byte never crosses a page), and thread
//     t loads blocks t, t + 256, ... with one buffer load each, all in
//     flight at once; several workgroups share a CU, so one row's loads
//     overlap the others' work;
//   * elements outside the row (and blocks past its end, read as zeros by the
//     clipped buffer view) become -inf, which changes neither the maximum,
//     the flag nor the survivors;
//   * each thread takes the maximum of its elements and the NaN / +inf flag
//     (packed 16-bit integer max/min over the raw patterns for 16-bit rows);
//     theta is the M-th largest of the 256 thread maxima, so at least M
//     elements are >= theta;
//   * the survivors (finite, allowed, x >= theta) are taken from the
//     registers; each survivor's rank among them (a count of the survivors
//     before it) places it in the shortlist, every thread ranking some.
//
// A row with NaN or +inf keeps no shortlist (the select pass reads such a row
// in full), as in the other row passes.
#include <hip/hip_runtime.h>

#include "row_helpers.hpp"

namespace dbs_hip {

namespace {

constexpr int kLpThreads = 256;
constexpr int kLpMaxBlocks = 40;  // 16-byte blocks per thread, at most
constexpr int kLpBlockCap = 512;  // blocks holding survivors, at most (else the row is read in full)

// Element i of a block as f32. binary16 goes through the hardware conversion,
// exact for every finite value and the infinities (denormals are kept); a NaN
// never reaches a shortlist (the row is flagged and read in full instead), so
// its payload does not matter here.
template <int DT>
__device__ __forceinline__ float element_of(const v4u32& d, int i) {
    if constexpr (DT == 0) {
        return bits_f32(d[i]);
    } else if constexpr (DT == 1) {
        const uint16_t h = static_cast<uint16_t>((d[i >> 1] >> (16 * (i & 1))) & 0xffffu);
        return static_cast<float>(__builtin_bit_cast(_Float16, h));
    } else {
        return pattern_value<DT>((d[i >> 1] >> (16 * (i & 1))) & 0xffffu);
    }
}

template <int DT>
__device__ __forceinline__ void set_neg_inf(v4u32& d, int i) {
    if constexpr (DT == 0) {
        d[i] = 0xff800000u;
    } else {
        const uint32_t ninf = DT == 1 ? 0xfc00u : 0xff80u;
        const int sh = 16 * (i & 1);
        d[i >> 1] = (d[i >> 1] & ~(0xffffu << sh)) | (ninf << sh);
    }
}

// Loads the 16-byte blocks of row r (thread t: blocks t, t + 256, ...) into
// d, returning the elements by which the first block starts before the row.
// Not valid (no row left): the same loads through an empty buffer view, which
// return zeros and touch no memory, so the loads never sit under a branch.
// Blocks C0 .. C1 - 1 only (the row is loaded in two parts).
template <int DT, int C, int C0 = 0, int C1 = C>
__device__ __forceinline__ int load_row(const DecodeParams& p, int64_t r, bool valid, int tid, v4u32 (&d)[C]) {
    constexpr int esz = DT == 0 ? 4 : 2;
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(p.x) + static_cast<uintptr_t>(valid ? r : 0) * p.V * esz;
    const int lead = static_cast<int>(a0 & 15u);
    const int nblk = valid ? (lead + p.V * esz + 15) >> 4 : 0;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(a0 - lead), 0, 16 * nblk, 0x00020000);
#pragma unroll
    for (int c = C0; c < C1; ++c) d[c] = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * tid, 4096 * c, kRowLoadPolicy);
    return lead / esz;
}

// Bytes of a token mask of V entries (null: none) for tokens v0 .. v0 + N - 1,
// through a buffer view of the mask: tokens outside [0, V), and every token
// of an absent mask, read 0 without touching memory. The loads are left
// outstanding (no branch around them): the caller pins the bytes where it
// wants to wait for them.
template <int N>
__device__ __forceinline__ void load_mask_bytes(const uint8_t* base, int v0, int V, uint32_t (&by)[N]) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, base ? V : 0, 0x00020000);
#pragma unroll
    for (int i = 0; i < N; ++i) by[i] = __builtin_amdgcn_raw_buffer_load_b8(rs, v0 + i, 0, 0);
}

// Whether token v ends a hypothesis of an example whose EOS token (with
// per-example EOS tokens) is eos_b.
__device__ __forceinline__ bool is_eos_given(const DecodeParams& p, int eos_b, int32_t v) {
    if (!p.eos_pe) return in_eos_set(p, v);
    return eos_b >= 0 && (v == eos_b || in_eos_set(p, v));
}

// The next row's EOS masking and EOS token (ticket thread; the row pass's
// loads of the current row have landed, so these waits cost only themselves).
__device__ __forceinline__ void next_row_options(const DecodeParams& p, int64_t rows, const RowSlot& slot, int& mask_eos,
                                                 int& eos_b) {
    mask_eos = 0;
    eos_b = -1;
    if (slot.r < rows) {
        mask_eos = slot.len < min_length_of(p, slot.b) ? 1 : 0;
        if (p.eos_pe) eos_b = gload(p.eos_pe, slot.b);
    }
}

// Persistent: a workgroup takes rows in turn (tickets in the overlapped
// decode, else its own stride), and issues the loads of its next row as soon
// as the current row's blocks that can hold survivors are copied to LDS, so
// those loads are in flight while the survivors are scanned, ranked and
// published; the last kLate blocks go out after the publishing, leaving their
// registers to the scan (three workgroups per CU at 32 blocks per thread).
// Barriers after that point order LDS only (lds_barrier), which keeps the
// loads outstanding across them.
template <int DT, int C>
__global__ __launch_bounds__(kLpThreads) __attribute__((amdgpu_waves_per_eu(C <= 32 ? 3 : 1))) void row_logprob_kernel(DecodeParams p, int64_t rows) {
    __shared__ uint64_t s_key[kSurvivorCap];
    __shared__ float s_x[kSurvivorCap];
    __shared__ __align__(16) uint32_t s_tkey[kLpThreads];
    __shared__ v4u32 s_blk[kLpBlockCap];
    __shared__ int s_blk_v0[kLpBlockCap];
    __shared__ RowSlot s_slot;
    __shared__ int s_slot_mask_eos;
    __shared__ int s_slot_eos;
    __shared__ int s_count;
    __shared__ int s_nblk;
    __shared__ int s_bad;
    __shared__ float s_theta;
    __shared__ float s_bound;

    constexpr int kTicketThread = 64;  // takes the tickets (a wavefront idle while wavefront 0 selects theta)
    const int tid = static_cast<int>(threadIdx.x);
    const int V = p.V;
    const int M = p.M;
    constexpr int esz = DT == 0 ? 4 : 2;
    constexpr int epb = 16 / esz;  // elements per block
    const bool coherent = p.step_done != nullptr;

    int64_t q = 0;  // processing index (kTicketThread's)
    if (tid == kTicketThread) {
        q = first_ticket(p);
        int b0 = 0, len0 = 0;
        s_slot.r = find_read_row(p, rows, q, b0, len0);
        s_slot.b = b0;
        s_slot.len = len0;
        next_row_options(p, rows, s_slot, s_slot_mask_eos, s_slot_eos);
        s_count = 0;
        s_nblk = 0;
        s_bad = 0;
    }
    __syncthreads();
    int b, len_unused;
    int64_t r = read_row_slot(s_slot, b, len_unused);
    bool mask_eos = s_slot_mask_eos != 0;
    int eos_b = s_slot_eos;
    v4u32 d[C];
    int lead_e = load_row<DT, C>(p, r, r < rows, tid, d);

    while (r < rows) {

        // Elements outside the row become -inf.
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int v0 = (c * kLpThreads + tid) * epb - lead_e;
            if (v0 < 0 || v0 + epb > V) {
#pragma unroll
                for (int i = 0; i < epb; ++i)
                    if (v0 + i < 0 || v0 + i >= V) set_neg_inf<DT>(d[c], i);
            }
        }

        // Thread maximum over x < +inf, its order key, and the NaN / +inf flag.
        float tmax = -kInf;
        uint32_t tkey;
        bool bad = false;
        if constexpr (DT == 0) {
#pragma unroll
            for (int c = 0; c < C; ++c) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float x = bits_f32(d[c][i]);
                    bad = bad || __builtin_amdgcn_classf(x, 0x203);  // sNaN, qNaN, +inf
                    tmax = fmaxf(tmax, x);
                }
            }
            tkey = ordered_key(tmax);
        } else {
            // Signed max/min and unsigned max of the raw patterns: the largest
            // value is the largest non-negative pattern, else the smallest
            // (most negative) signed one; a signed max >= +inf's pattern flags
            // +inf or a positive NaN, an unsigned max above -inf's a negative NaN.
            uint32_t smax = 0x80008000u, smin = 0x7fff7fffu, umax = 0u;
#pragma unroll
            for (int c = 0; c < C; ++c) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    smax = pk_max_i16(smax, d[c][i]);
                    smin = pk_min_i16(smin, d[c][i]);
                    umax = pk_max_u16(umax, d[c][i]);
                }
            }
            const int pos_inf = DT == 1 ? 0x7c00 : 0x7f80;
            const uint32_t neg_inf = DT == 1 ? 0xfc00u : 0xff80u;
            int best = -32768;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int16_t hmax = static_cast<int16_t>(smax >> (16 * h));
                const int16_t hmin = static_cast<int16_t>(smin >> (16 * h));
                bad = bad || hmax >= pos_inf || ((umax >> (16 * h)) & 0xffffu) > neg_inf;
                best = max(best, key16(static_cast<uint16_t>(hmax >= 0 ? hmax : hmin)));
            }
            tmax = pattern_value<DT>(key_pattern(best));
            tkey = static_cast<uint32_t>(best + 32768);  // the signed key, biased to 16 unsigned bits
        }
        s_tkey[tid] = tkey;
        if (__any(bad) && (tid & 63) == 0) s_bad = 1;
        __syncthreads();

        // theta = the M-th largest thread maximum (wavefront 0), so at least M
        // elements are >= theta; meanwhile kTicketThread finds the next row.
        const bool any_bad = s_bad != 0;
        if (tid < 64) {
            if (M > 0 && !any_bad) {
                int tq = tid;  // (recomputed, not kept live across the loop)
                asm volatile("" : "+v"(tq));
                const uint4 kk = reinterpret_cast<const uint4*>(s_tkey)[tq];
                const uint32_t k4[4] = {kk.x, kk.y, kk.z, kk.w};
                float th;
                if constexpr (DT == 0) {
                    th = key_value(mth_largest_key<32>(k4, M));
                } else {
                    th = pattern_value<DT>(key_pattern(static_cast<int>(mth_largest_key<16>(k4, M)) - 32768));
                }
                if (tid == 0) s_theta = th;
            }
        } else if (tid == kTicketThread) {
            s_nblk = 0;
            s_count = 0;
            publish_next_row(p, rows, q, s_slot);
            next_row_options(p, rows, s_slot, s_slot_mask_eos, s_slot_eos);
        }
        __syncthreads();
        if (tid == kTicketThread) s_bad = 0;  // every thread has read it
        const float theta = (M > 0 && !any_bad) ? s_theta : -kInf;
        const bool full = M > 0 && !(theta > -kInf);  // no shortlist: every element would survive

        // Blocks that can hold survivors (maximum >= theta) are copied to LDS.
        if (M > 0 && !full && tmax >= theta) {
            // (an opaque copy: the block starts are recomputed here rather than
            // kept in registers from the edge test above)
            int vt = tid * epb - lead_e;
            asm volatile("" : "+v"(vt));
#pragma unroll
            for (int c = 0; c < C; ++c) {
                float bm = -kInf;
#pragma unroll
                for (int i = 0; i < epb; ++i) bm = fmaxf(bm, element_of<DT>(d[c], i));
                if (bm >= theta) {
                    const int slot = atomicAdd(&s_nblk, 1);
                    if (slot < kLpBlockCap) {
                        s_blk[slot] = d[c];
                        s_blk_v0[slot] = vt + c * kLpThreads * epb;
                    }
                }
            }
        }
        __syncthreads();
        const int nblk_hit = s_nblk;
        const bool keep = M > 0 && !full && nblk_hit <= kLpBlockCap;

        // The banned bytes of this thread's first block, then the next row's
        // loads (the registers are free now), then the scan; the bytes are
        // waited for only after the next row's loads are issued.
        const bool mine = keep && tid < nblk_hit;  // a block to scan (the others read an empty view)
        const int v00 = mine ? s_blk_v0[tid] : 0;
        uint32_t ban_by[epb];  // the per-example mask, else the shared one
        load_mask_bytes<epb>(!mine ? nullptr : (p.banned_pe ? p.banned_pe + static_cast<int64_t>(b) * V : p.banned), v00,
                             V, ban_by);
        int bn;
        const int64_t rn = read_row_slot(s_slot, bn, len_unused);
        const bool mask_eos_n = s_slot_mask_eos != 0;
        const int eos_n = s_slot_eos;
        constexpr int kLate = C >= 16 ? 4 : 0;
        const int lead_n = load_row<DT, C, 0, C - kLate>(p, rn, rn < rows, tid, d);
#pragma unroll
        for (int e = 0; e < epb; ++e) asm volatile("" : "+v"(ban_by[e])::"memory");

        if (keep) {
            for (int i = tid; i < nblk_hit; i += kLpThreads) {
                const v4u32 blk = s_blk[i];
                const int v0 = s_blk_v0[i];
                uint32_t ban = 0;
                if (i == tid && !(p.banned_pe && p.banned)) {
#pragma unroll
                    for (int e = 0; e < epb; ++e) ban |= (ban_by[e] != 0u ? 1u : 0u) << e;
                } else {  // both masks, or a second block of this thread (rare): read here
#pragma unroll
                    for (int e = 0; e < epb; ++e)
                        ban |= (v0 + e >= 0 && v0 + e < V && static_masked(p, b, v0 + e, false) ? 1u : 0u) << e;
                }
#pragma unroll
                for (int e = 0; e < epb; ++e) {
                    const float x = element_of<DT>(blk, e);
                    const int v = v0 + e;
                    if (x >= theta && x < kInf && !((ban >> e) & 1u) && !(mask_eos && is_eos_given(p, eos_b, v))) {
                        const int slot = atomicAdd(&s_count, 1);
                        if (slot < kSurvivorCap) {
                            s_key[slot] = survivor_key(x, v);
                            s_x[slot] = x;
                        }
                    }
                }
            }
        }
        lds_barrier();

        // The shortlist: each survivor's rank is the number of survivors
        // before it (keys are distinct); ranks below M are written in place,
        // rank M is the bound on the rest.
        const int n = s_count;
        const bool listed = keep && n <= kSurvivorCap;
        if (listed) {
            ShortEntry* out = p.shortlist + r * M;
            for (int i = tid; i < n; i += kLpThreads) {
                const uint64_t ki = s_key[i];
                int rank = 0;
                int j = 0;
                for (; j + 4 <= n; j += 4) {
                    const uint64_t k0 = s_key[j], k1 = s_key[j + 1], k2 = s_key[j + 2], k3 = s_key[j + 3];
                    rank += static_cast<int>(k0 > ki) + static_cast<int>(k1 > ki) + static_cast<int>(k2 > ki) +
                            static_cast<int>(k3 > ki);
                }
                for (; j < n; ++j) rank += static_cast<int>(s_key[j] > ki);
                if (rank < M) {
                    const int32_t tok = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(ki & 0xffffffffu));
                    publish_entry(out, rank, s_x[i], tok, coherent);
                } else if (rank == M) {
                    s_bound = s_x[i];
                }
            }
        }
        lds_barrier();
        if (tid < 64) {
            RowInfo info;
            info.lse = 0.0f;
            info.invalid = any_bad ? 1u : 0u;
            info.bound = -kInf;
            info.count = 0;
            if (M > 0) {
                if (listed) {
                    info.count = n < M ? n : M;
                    info.bound = n > M ? s_bound : theta;
                } else {
                    info.count = -1;
                }
            }
            if (tid == 0) publish_rowinfo(p.rowinfo + r, info, coherent);
            signal_row_done(p, r, tid);
        }
        if constexpr (kLate > 0) load_row<DT, C, C - kLate, C>(p, rn, rn < rows, tid, d);
        r = rn;
        b = bn;
        mask_eos = mask_eos_n;
        eos_b = eos_n;
        lead_e = lead_n;
    }
}

// Blocks per thread for a row of V elements (the first block may start up to
// 15 bytes before the row).
int logprob_blocks(const DecodeParams& p) {
    const int64_t esz = p.dtype == 0 ? 4 : 2;
    const int64_t nblk = (15 + static_cast<int64_t>(p.V) * esz + 15) / 16;
    return static_cast<int>((nblk + kLpThreads - 1) / kLpThreads);
}

}  // namespace

bool row_logprob_eligible(const DecodeParams& p) {
    if (p.from_logits) return false;
    if (p.M > 256) return false;
    return logprob_blocks(p) <= kLpMaxBlocks;
}

namespace {

int g_lp_cus[64];

// Resident workgroups of one instantiation per CU (every gfx950 the same).
template <int DT, int C>
int lp_per_cu() {
    static const int n = [] {
        int blocks = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, reinterpret_cast<const void*>(&row_logprob_kernel<DT, C>),
                                                         kLpThreads, 0) != hipSuccess || blocks < 1)
            blocks = 1;
        return blocks;
    }();
    return n;
}

template <int DT, int C>
hipError_t launch_lp(const DecodeParams& p, int64_t rows, int cus, hipStream_t stream) {
    const int64_t slots = static_cast<int64_t>(cus) * lp_per_cu<DT, C>();
    const int64_t grid = rows < slots ? rows : slots;
    hipLaunchKernelGGL((row_logprob_kernel<DT, C>), dim3(static_cast<unsigned>(grid)), dim3(kLpThreads), 0, stream, p,
                       rows);
    return hipGetLastError();
}

}  // namespace

// One workgroup per resident slot (at most one per row); beside a select
// pass that holds its CUs, on the CUs left.
hipError_t launch_row_logprob(const DecodeParams& p, int64_t rows, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const int need = logprob_blocks(p);
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    if (g_lp_cus[device] == 0) {
        int cus = 0;
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
        if (e != hipSuccess) return e;
        g_lp_cus[device] = cus > 0 ? cus : 1;
    }
    const int held = p.select_hold ? p.reserve_cus : 0;
    const int cus = g_lp_cus[device] - held > 0 ? g_lp_cus[device] - held : 1;
#define DBS_LP_CASE(CB)                                                       \
    if (need <= CB) {                                                         \
        if (p.dtype == 0) return launch_lp<0, CB>(p, rows, cus, stream);      \
        if (p.dtype == 1) return launch_lp<1, CB>(p, rows, cus, stream);      \
        return launch_lp<2, CB>(p, rows, cus, stream);                        \
    }
    DBS_LP_CASE(2)
    DBS_LP_CASE(4)
    DBS_LP_CASE(8)
    DBS_LP_CASE(12)
    DBS_LP_CASE(16)
    DBS_LP_CASE(20)
    DBS_LP_CASE(24)
    DBS_LP_CASE(28)
    DBS_LP_CASE(32)
    DBS_LP_CASE(40)
#undef DBS_LP_CASE
    return hipErrorInvalidValue;
}

}  // namespace dbs_hip
