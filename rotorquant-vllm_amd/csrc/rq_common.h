// Shared helpers for the gfx950 RotorQuant kernels: error reporting, dtype
// conversion, packed-slot offsets and the in-register codebook lookup.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/rq_abi.h"

namespace rq {

// ---------------------------------------------------------------------------
// Error reporting (thread-local message, returned status)
// ---------------------------------------------------------------------------
void set_error(const char *fmt, ...);

#define RQ_CHECK_ARG(cond, ...)            \
    do {                                   \
        if (!(cond)) {                     \
            ::rq::set_error(__VA_ARGS__);  \
            return RQ_EINVAL;              \
        }                                  \
    } while (0)

int check_launch(const char *what);

// ---------------------------------------------------------------------------
// Packed slot layout: [K idx | K norms | V idx | V norms | pad]
// (reference: src/rotorquant_vllm/vllm/rq_backend.py:155-188, :482-490)
// ---------------------------------------------------------------------------
struct SlotLayout {
    int32_t H, D, half;
    int32_t k_idx, k_norm, v_idx, v_norm, payload;
    __host__ __device__ SlotLayout(int32_t h, int32_t d) : H(h), D(d), half(d / 2) {
        k_idx = 0;
        k_norm = H * half;
        v_idx = k_norm + 4 * H;
        v_norm = v_idx + H * half;
        payload = v_norm + 4 * H;
    }
};

typedef __attribute__((address_space(3))) uint8_t lds_u8;

__device__ __forceinline__ uint32_t lds_addr(const uint8_t *p) { return (uint32_t)(size_t)(lds_u8 *)p; }

// Max / sum over lanes l, l^16, l^32, l^48 (the four 16-lane rows) with the
// gfx950 row-swap permutes: swapping a register with itself leaves lane l
// holding {x[l], x[l^32]} (resp. {x[l], x[l^16]}) in the two results.
__device__ __forceinline__ float rows_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// Direct global -> LDS copies, issued as inline assembly so that the compiler
// neither waits for them before unrelated LDS accesses nor counts them: the
// kernel waits for them itself with s_waitcnt vmcnt.  Lane l writes its bytes
// at LDS address m0 + l * size (m0 = wave-uniform destination).
//   copy16:  16 bytes from the uniform base `src` + per-lane 32-bit offset.
//   copy16v: 16 bytes from a per-lane address.
//   copy4s:  4 bytes from the uniform base `src` + per-lane 32-bit offset.
//   copy4:   4 bytes from a per-lane address.
__device__ __forceinline__ void copy16(const uint8_t *src, uint32_t voff, uint32_t dst) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(src), "s"(dst)
                 : "memory", "m0");
}
__device__ __forceinline__ void copy16v(const uint8_t *src, uint32_t dst) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(dst) : "memory", "m0");
}
__device__ __forceinline__ void copy4s(const uint8_t *src, uint32_t voff, uint32_t dst) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(src), "s"(dst)
                 : "memory", "m0");
}
__device__ __forceinline__ void copy4(const uint8_t *src, uint32_t dst) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(dst) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_copies() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Compute units of the current device (cached per device).
inline int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

inline int32_t next_pow2_i32(int32_t n) {
    int32_t p = 1;
    while (p < n) p <<= 1;
    return p;
}

// ---------------------------------------------------------------------------
// Scalar conversions (round to nearest even)
// ---------------------------------------------------------------------------

// Hides a value from the optimiser (no instruction emitted).  Used where an
// fp32 product must be rounded to fp32 before a 16-bit cast: without it the
// backend folds multiply + cast into one v_fma_mix with a +0 addend, which
// rounds once instead of twice and turns -0 into +0.
__device__ __forceinline__ float opaque(float x) {
    asm volatile("" : "+v"(x));
    return x;
}
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    // gfx950 converts with v_cvt_pk_bf16_f32 (round to nearest even).
    __bf16 b = (__bf16)f;
    uint16_t s;
    __builtin_memcpy(&s, &b, 2);
    return s;
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
    _Float16 h;
    uint16_t s = (uint16_t)b;
    __builtin_memcpy(&h, &s, 2);
    return (float)h;
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;
    uint16_t s;
    __builtin_memcpy(&s, &h, 2);
    return s;
}

template <int DT> struct Elem;
template <> struct Elem<RQ_DTYPE_F16> {
    using storage = uint16_t;
    static __device__ __forceinline__ float to_f32(uint32_t b) { return f16_bits_to_f32(b); }
    static __device__ __forceinline__ uint32_t from_f32(float f) { return f32_to_f16_bits(f); }
};
template <> struct Elem<RQ_DTYPE_BF16> {
    using storage = uint16_t;
    static __device__ __forceinline__ float to_f32(uint32_t b) { return bf16_bits_to_f32(b); }
    static __device__ __forceinline__ uint32_t from_f32(float f) { return f32_to_bf16_bits(f); }
};
template <> struct Elem<RQ_DTYPE_F32> {
    using storage = float;
};

// ---------------------------------------------------------------------------
// Codebook lookup in registers with v_perm_b32.
//
// A 16-bit codebook entry (bf16 or f16 bits of a centroid) is split into its
// low and high byte.  For 8 entries the 8 low bytes live in two dwords (lo0:
// entries 0-3, lo1: entries 4-7) and the 8 high bytes likewise; v_perm with a
// selector whose bytes are indices 0..7 then gathers 4 low (or high) bytes at
// once.  16-entry codebooks use two such tables and merge on index bit 3.
// ---------------------------------------------------------------------------
struct Table16 {
    uint32_t lo[4];  // low bytes of entries 0..15
    uint32_t hi[4];  // high bytes of entries 0..15
};

__device__ __forceinline__ uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
    return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

// sel: four selector bytes, each an index 0..(2^BITS - 1).  Returns the four
// looked-up 16-bit values as two dwords: .x = [v0 | v1 << 16], .y = [v2 | v3 << 16].
template <int BITS>
__device__ __forceinline__ uint2 lookup4(const Table16 &t, uint32_t sel) {
    uint32_t L, Hh;
    if constexpr (BITS == 3) {
        L = perm(t.lo[1], t.lo[0], sel);
        Hh = perm(t.hi[1], t.hi[0], sel);
    } else {
        uint32_t s7 = sel & 0x07070707u;
        // 0xFF in every byte whose index has bit 3 set.
        uint32_t m = ((sel >> 3) & 0x01010101u) * 0xFFu;
        uint32_t la = perm(t.lo[1], t.lo[0], s7), lb = perm(t.lo[3], t.lo[2], s7);
        uint32_t ha = perm(t.hi[1], t.hi[0], s7), hb = perm(t.hi[3], t.hi[2], s7);
        L = (la & ~m) | (lb & m);
        Hh = (ha & ~m) | (hb & m);
    }
    return make_uint2(perm(Hh, L, 0x05010400u),   // [L0, H0, L1, H1]
                      perm(Hh, L, 0x07030602u));  // [L2, H2, L3, H3]
}

}  // namespace rq
