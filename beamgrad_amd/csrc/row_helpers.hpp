// SPDX-License-Identifier: MIT
//
// Helpers of the row passes that keep 16-bit rows on chip: packed 16-bit
// integer operations, buffer views, LDS-only barriers, the 16-bit pattern
// keys, the bfloat16 term table bounds and the histogram radix select.
#pragma once

#include <hip/hip_runtime.h>

#include "device_common.hpp"

namespace dbs_hip {

constexpr int kLutHalf = 4096;  // bfloat16 term-table slots per sign
// Cache policy of the row passes' streamed row loads: nt (non-temporal).
// Every row is read once per pass; on MI355X a read-only stream of 16-byte
// loads reaches 6.6 TB/s with it against 5.9 TB/s without.
constexpr int kRowLoadPolicy = 2;

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
__device__ __forceinline__ uint32_t pk_add_u16(uint32_t a, uint32_t b) {  // wrapping
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2u16, a) + __builtin_bit_cast(v2u16, b));
}
__device__ __forceinline__ uint32_t pk_sign_fill_i16(uint32_t a) {
    const v2i16 fifteen = {15, 15};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2i16, a) >> fifteen);
}
__device__ __forceinline__ uint32_t pk_shl2_u16(uint32_t a) {
    const v2u16 two = {2, 2};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2u16, a) << two);
}

// Buffer view of one row (bytes [0, nbytes)): loads past its end return
// zeros instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_buffer(const uint16_t* row, int nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(row), 0, nbytes, 0x00020000);
}

typedef unsigned int v2u32 __attribute__((ext_vector_type(2)));
typedef unsigned int v4u32 __attribute__((ext_vector_type(4)));


template <int DT>
__device__ __forceinline__ float pattern_value(uint32_t h) {
    return DT == 1 ? half_to_f32(static_cast<uint16_t>(h)) : bf16_to_f32(static_cast<uint16_t>(h));
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

// Transposes one chunk: lane L holds 16 bytes = lanes 8 (L % 8) .. + 7 of
// stripe L / 8; it gets back its own lane L of the 8 stripes, packed two
// stripes per register (lower stripe in the low half). The chunk goes through
// the wavefront's 1 KB slot, (stripe i, lane L) at byte 128 i + 2 L, read back
// with two transposing reads: within each 16-lane group, lane i receives
// element i % 4 of the 8 bytes addressed by lanes 4 k + i / 4 (k = 0..3), so
// lane L = 16 G + a addresses (stripe 4 h + a / 4, lanes 16 G + 4 (a % 4) ..).
// The write and the reads go through the compiler's LDS operations, so the
// next chunk's transpose can start before this one's results are used.
__device__ __forceinline__ void transpose_chunk(unsigned char* slot, int L, uint32_t x0, uint32_t x1, uint32_t x2,
                                                uint32_t x3, uint32_t (&R)[4]) {
    typedef short v4i16 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) unsigned char lds_u8;
    const int G = L >> 4, a = L & 15;
    lds_u8* base = (lds_u8*)slot;
    *reinterpret_cast<__attribute__((address_space(3))) v4u32*>(base + 16 * L) = v4u32{x0, x1, x2, x3};
    lds_u8* rd = base + 128 * (a >> 2) + 32 * G + 8 * (a & 3);
    const v4i16 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<__attribute__((address_space(3))) v4i16*>(rd));
    const v4i16 t1 =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<__attribute__((address_space(3))) v4i16*>(rd + 512));
    const v2u32 u0 = __builtin_bit_cast(v2u32, t0), u1 = __builtin_bit_cast(v2u32, t1);
    R[0] = u0.x;
    R[1] = u0.y;
    R[2] = u1.x;
    R[3] = u1.y;
}

// The term table with a fixed base: slot k >= 1 of each sign holds magnitude
// kFixedBase - 1 + k (the bfloat16 pattern 0x3300 is 2^-25), slot 0 every
// smaller magnitude. The slot of a pattern then does not depend on the row,
// so it can be computed as soon as the pattern is in registers. It fits a row
// with maximum m when 1 <= m (every |x| < 2^-25 <= half an ulp of m gives
// fl(x - m) = -m, slot 0's exp(-m)) and m's pattern lies below the last slot
// (a positive pattern never clamps; +inf and +NaN clamp to the last positive
// slot, which holds 0, as do -inf, -NaN and every magnitude >= 127.5 in the
// last negative slot: exp(-127.5 - m) is 0).
constexpr uint32_t kFixedBase = 0x3300u;
__device__ __forceinline__ bool table_fits_fixed(float m) {
    if (!(m >= 1.0f && m < kInf)) return false;
    const uint32_t mp = f32_bits(m) >> 16;
    return mp < kFixedBase - 1 + (kLutHalf - 1);
}

// Slots in the fixed-base table of a register's two bfloat16 patterns (low
// half, high half): slot = min(max(magnitude - (base - 1), 0), 4095), plus
// 4096 for a negative pattern. Five packed 16-bit operations; a lookup takes
// the byte offset with one shift of its half (slot * 4).
__device__ __forceinline__ uint32_t term_slots(uint32_t R) {
    uint32_t idx = pk_sub_sat_u16(R & 0x7fff7fffu, (kFixedBase - 1u) * 0x10001u);
    idx = pk_min_u16(idx, 0x0fff0fffu);
    return idx | ((R >> 3) & 0x10001000u);
}

// Inverse of key16.
__device__ __forceinline__ uint32_t key_pattern(int key) {
    return static_cast<uint16_t>(key < 0 ? (key ^ 0x7fff) : key);
}

// The maximum over a wavefront's 64 lanes (every lane gets it).
__device__ __forceinline__ int wave_max_int(int x) {
    const int lo = static_cast<int>(0x80000000u);
    x = max(x, __builtin_amdgcn_update_dpp(lo, x, 0x111, 0xf, 0xf, false));
    x = max(x, __builtin_amdgcn_update_dpp(lo, x, 0x112, 0xf, 0xf, false));
    x = max(x, __builtin_amdgcn_update_dpp(lo, x, 0x114, 0xf, 0xf, false));
    x = max(x, __builtin_amdgcn_update_dpp(lo, x, 0x118, 0xf, 0xf, false));
    x = max(x, __builtin_amdgcn_update_dpp(lo, x, 0x142, 0xa, 0xf, false));
    x = max(x, __builtin_amdgcn_update_dpp(lo, x, 0x143, 0xc, 0xf, false));
    return __builtin_amdgcn_readlane(x, 63);
}

// Over 256 bins taken in descending order, the bin holding the target-th
// largest count-weighted key (1-based; the bins hold at least target keys),
// and how many keys lie in the bins above it. One wavefront, every lane gets
// the answer.
__device__ __forceinline__ void hist_select(const int* hist, int target, int lane, int& bin, int& above) {
    const int4 h = *reinterpret_cast<const int4*>(hist + 252 - 4 * lane);  // bins 252-4l .. 255-4l
    const int c0 = h.w, c1 = h.z, c2 = h.y, c3 = h.x;                     // descending
    const int sum = c0 + c1 + c2 + c3;
    const int incl = wave_inclusive_sum(sum);
    const int excl = incl - sum;
    const uint64_t mine = __ballot(excl < target && target <= incl);
    const int src = __ffsll(static_cast<long long>(mine)) - 1;
    int b = 255 - 4 * lane, a = excl;
    if (a + c0 < target) {
        a += c0;
        --b;
        if (a + c1 < target) {
            a += c1;
            --b;
            if (a + c2 < target) {
                a += c2;
                --b;
            }
        }
    }
    bin = __shfl(b, src);
    above = __shfl(a, src);
}

// Row sequence of a persistent row-pass workgroup. Thread 0 finds the rows
// (the workgroup's stride, or tickets in the overlapped decode) and publishes
// them in LDS slots; every wavefront reads a slot after a barrier.
struct RowSlot {
    long long r;
    int b, len;
};

// TICKETS false: the workgroup's fixed stride even where tickets are handed
// out (a kernel whose rows all cost the same).
template <bool TICKETS = true>
__device__ __forceinline__ int64_t next_index(const DecodeParams& p, int64_t q) {
    return TICKETS ? take_ticket(p, q, gridDim.x) : q + gridDim.x;
}

template <bool TICKETS = true>
__device__ __forceinline__ int64_t first_ticket(const DecodeParams& p) {
    return (TICKETS && p.row_ticket) ? take_ticket(p, 0, 0) : static_cast<int64_t>(blockIdx.x);
}

// From processing index q on, the first row the search reads (q is left at
// it), or rows when none is left.
template <bool TICKETS = true>
__device__ __forceinline__ int64_t find_read_row(const DecodeParams& p, int64_t rows, int64_t& q, int& b, int& len) {
    while (q < rows) {
        const int64_t rr = row_of_ticket(p, q);
        if (row_is_read(p, rr, b, len)) return rr;
        q = next_index<TICKETS>(p, q);
    }
    return rows;
}

// Thread 0: the row after processing index q (advanced) into slot.
template <bool TICKETS = true>
__device__ __forceinline__ void publish_next_row(const DecodeParams& p, int64_t rows, int64_t& q, RowSlot& slot) {
    int b = 0, len = 0;
    int64_t rr = rows;
    if (q < rows) {
        q = next_index<TICKETS>(p, q);
        rr = find_read_row<TICKETS>(p, rows, q, b, len);
    }
    slot.r = rr;
    slot.b = b;
    slot.len = len;
}

// Every lane: a published row (kept in scalar registers).
__device__ __forceinline__ int64_t read_row_slot(const RowSlot& slot, int& b, int& len) {
    const long long rr = slot.r;
    b = __builtin_amdgcn_readfirstlane(slot.b);
    len = __builtin_amdgcn_readfirstlane(slot.len);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(rr));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<unsigned long long>(rr) >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

}  // namespace dbs_hip
