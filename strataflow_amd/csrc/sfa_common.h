// sfa_common.h - shared device/host helpers of the gfx950 paged-KV attention
// library.  Wave64 only (CDNA4); no other target is built.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sfa.h"

namespace sfa {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef int intx4 __attribute__((ext_vector_type(4)));
typedef int intx16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;
constexpr int kTile = 32;    // positions per wave tile in decode
constexpr int kQK = 32;      // Q8_0 block length
constexpr int kQ8Bytes = 34; // sizeof(block_q8_0)
// Word 3 of a raw (unformatted, stride 0) buffer resource on gfx9-family
// parts: data format 32 bits, no swizzle, no index stride.  num_records then
// counts bytes and a load past it returns zeros instead of reading memory.
constexpr int kBufferRsrcWord3 = 0x00020000;

// Row bytes of one (position, kv head) row for a cache type; 0 if unsupported.
__host__ __device__ inline int row_bytes_of(int kv_type, int head_dim) {
    switch (kv_type) {
    case SFA_KV_F32: return head_dim * 4;
    case SFA_KV_F16: return head_dim * 2;
    case SFA_KV_Q8_0: return (head_dim / kQK) * kQ8Bytes;
    default: return 0;
    }
}

// Resolves a page-table entry to the base address of that page in the device
// pool (id >= 0) or the cold pool (id <= -2).  Returns nullptr for -1 or an id
// outside the pool, so a bad table never turns into an out-of-bounds read.
__device__ inline const uint8_t *page_base(int32_t id, const uint8_t *pool, int n_pages,
                                           const uint8_t *cold, int n_cold,
                                           int64_t page_bytes) {
    if (id >= 0) {
        if (id >= n_pages || pool == nullptr) return nullptr;
        return pool + (int64_t)id * page_bytes;
    }
    if (id <= -2) {
        const int64_t c = -2 - (int64_t)id;
        if (c >= n_cold || cold == nullptr) return nullptr;
        return cold + c * page_bytes;
    }
    return nullptr;
}

// ds_read_b64_tr_b16: with every lane of a 16-lane group addressing an
// 8-byte chunk of four 16-bit values, lane i of the group receives value i%4
// of the chunks addressed by lanes i/4, 4 + i/4, 8 + i/4, 12 + i/4 (in that
// order).  The address must be 8-byte aligned.
__device__ inline half4 tr16_read(const uint8_t *lds_addr) {
    typedef short short4_t __attribute__((ext_vector_type(4)));
    const auto p = (__attribute__((address_space(3))) short4_t *)(
        (__attribute__((address_space(3))) uint8_t *)(lds_addr));
    const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(p);
    return __builtin_bit_cast(half4, v);
}

// 16- and 4-byte global loads from 4-byte aligned addresses (Q8_0 rows are
// only 4-byte aligned; global loads need dword alignment on this target).
__device__ inline intx4 load16_a4(const uint8_t *p) {
    intx4 v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, 4), 16);
    return v;
}
__device__ inline uint32_t load4_a4(const uint8_t *p) {
    return *reinterpret_cast<const uint32_t *>(__builtin_assume_aligned(p, 4));
}

// Page ids of 64 consecutive logical pages of one sequence, one per lane, so
// that a tile's page id is a v_readlane instead of a dependent memory load on
// every tile (a wave's tiles rarely leave one window; when they do, the
// window moves).  `lp` must be wave-uniform.
struct PageWindow {
    int base;
    int32_t ids;
    // The load is unconditional (a clamped index, then a select): a load in a
    // branch makes the compiler's wait at the join count every later load too.
    __device__ inline void load(const int32_t *pt, int max_pages, int first, int lane) {
        base = first;
        const int lp = first + lane;
        const int32_t id = pt[lp < max_pages ? lp : max_pages - 1];
        ids = lp < max_pages ? id : -1;
    }
    __device__ inline int32_t get(const int32_t *pt, int max_pages, int lp, int lane) {
        if (lp < base || lp >= base + kWave) load(pt, max_pages, lp, lane);
        return __builtin_amdgcn_readlane(ids, lp - base);
    }
};

// Cross-half exchange: value of lane (l ^ 32).
__device__ inline float xor32(float x) {
    return __shfl_xor(x, 32, 64);
}

// Both halves of x in every lane, by one v_permlane32_swap (a VALU op, no
// LDS round trip): lo = x of lane l % 32, hi = x of lane 32 + l % 32.  The
// builtin's pair is read by bytes: indexing its second element returned the
// first one with this compiler.
__device__ inline void swap_halves(float x, float &lo, float &hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x),
                                                    false, false);
    static_assert(sizeof(r) == 8, "two 32-bit lanes values");
    unsigned u0, u1;
    __builtin_memcpy(&u0, reinterpret_cast<const char *>(&r), 4);
    __builtin_memcpy(&u1, reinterpret_cast<const char *>(&r) + 4, 4);
    lo = __builtin_bit_cast(float, u0);
    hi = __builtin_bit_cast(float, u1);
}

// max(a, b, c) in one v_max3_f32.  fmaxf makes the compiler quiet signalling
// NaNs first (one more v_max per operand); for MFMA results and -INF masks
// that cannot occur, and the result is the same.
__device__ inline float max3_raw(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Value of another lane of the same 16-lane row, DPP control CTRL (all rows
// and banks enabled, every source lane inside the row).
template <int CTRL>
__device__ inline float dpp_row(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
__device__ inline float lane_val(float x, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

// Wave-wide max and sum (the same value in every lane): butterflies inside
// each 16-lane row (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror), then the four row results in a fixed order.
__device__ inline float wave_max(float x) {
    x = fmaxf(x, dpp_row<0xB1>(x));
    x = fmaxf(x, dpp_row<0x4E>(x));
    x = fmaxf(x, dpp_row<0x141>(x));
    x = fmaxf(x, dpp_row<0x140>(x));
    return fmaxf(fmaxf(lane_val(x, 0), lane_val(x, 16)), fmaxf(lane_val(x, 32), lane_val(x, 48)));
}
__device__ inline float wave_sum(float x) {
    x += dpp_row<0xB1>(x);
    x += dpp_row<0x4E>(x);
    x += dpp_row<0x141>(x);
    x += dpp_row<0x140>(x);
    return (lane_val(x, 0) + lane_val(x, 16)) + (lane_val(x, 32) + lane_val(x, 48));
}

}  // namespace sfa
