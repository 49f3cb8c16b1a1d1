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

// A caller-provided workspace smaller than the call needs: RQ_ENOSPACE.
#define RQ_CHECK_SPACE(cond, ...)          \
    do {                                   \
        if (!(cond)) {                     \
            ::rq::set_error(__VA_ARGS__);  \
            return RQ_ENOSPACE;            \
        }                                  \
    } while (0)

int check_launch(const char *what);

// ---------------------------------------------------------------------------
// Packed slot layout: [K idx | K norms | V idx | V norms | pad]
// (reference: src/rotorquant_vllm/vllm/rq_backend.py:155-188, :482-490).
// Index bytes per head: D / 2 (nibbles, the reference's layout) or, with the
// opt-in dense 3-bit layout, 3 D / 8 (see below).
// ---------------------------------------------------------------------------
struct SlotLayout {
    int32_t H, D, half;
    int32_t ib;  // index bytes per head
    int32_t k_idx, k_norm, v_idx, v_norm, payload;
    __host__ __device__ SlotLayout(int32_t h, int32_t d, bool dense3 = false)
        : H(h), D(d), half(d / 2), ib(dense3 ? 3 * d / 8 : d / 2) {
        k_idx = 0;
        k_norm = H * ib;
        v_idx = k_norm + 4 * H;
        v_norm = v_idx + H * ib;
        payload = v_norm + 4 * H;
    }
};

// ---------------------------------------------------------------------------
// Dense 3-bit index layout (opt-in; no counterpart in the reference, which
// lists 3-bit storage on its roadmap only).  The 32 indices i[0..31] of dims
// 32G .. 32G+31 of a head take 12 bytes, dwords A, B, C; byte k (k = 0..3):
//   A[k] = i[2k]    | i[2k+1] << 3  | (i[24+2k] & 3) << 6
//   B[k] = i[8+2k]  | i[9+2k] << 3  | (i[25+2k] & 3) << 6
//   C[k] = i[16+2k] | i[17+2k] << 3 | (i[24+2k] >> 2) << 6 | (i[25+2k] >> 2) << 7
// so that position w < 3 of the group (dims 8w .. 8w+7) reads like a nibble
// dword: one mask gives its even dims' indices one per byte (the selector a
// v_perm lookup takes), a shift and a mask its odd dims'; position 3 gathers
// its bits from the spare top bits of A, B and C.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ uint32_t d3_even(uint32_t x) { return x & 0x07070707u; }
__host__ __device__ __forceinline__ uint32_t d3_odd(uint32_t x) { return (x >> 3) & 0x07070707u; }
__host__ __device__ __forceinline__ uint32_t d3_even3(uint32_t a, uint32_t c) {
    return ((a >> 6) & 0x03030303u) | ((c >> 4) & 0x04040404u);
}
__host__ __device__ __forceinline__ uint32_t d3_odd3(uint32_t b, uint32_t c) {
    return ((b >> 6) & 0x03030303u) | ((c >> 5) & 0x04040404u);
}
// Nibble dword (byte k = i[8w+2k] << 4 | i[8w+2k+1]) of position w of a group.
__host__ __device__ __forceinline__ uint32_t d3_nibbles(uint32_t a, uint32_t b, uint32_t c, int w) {
    const uint32_t x = w == 0 ? a : (w == 1 ? b : c);
    const uint32_t e = w < 3 ? d3_even(x) : d3_even3(a, c);
    const uint32_t o = w < 3 ? d3_odd(x) : d3_odd3(b, c);
    return (e << 4) | o;
}
// Host check of an index_layout argument against head_dim and the codebook sizes.
inline int check_index_layout(int layout, int D, int n_k, int n_v) {
    RQ_CHECK_ARG(layout == RQ_INDEX_NIBBLE || layout == RQ_INDEX_DENSE3, "index_layout %d unknown", layout);
    if (layout == RQ_INDEX_DENSE3)
        RQ_CHECK_ARG(D % 32 == 0 && n_k <= 8 && n_v <= 8,
                     "the dense 3-bit layout needs head_dim %% 32 == 0 and at most 8 centroids / 7 boundaries "
                     "(head_dim %d, %d and %d)", D, n_k, n_v);
    return RQ_OK;
}

// The nibble dword of dims 8 dw .. 8 dw + 7 of a head whose index bytes start at
// p (4-byte aligned): a plain load, or the dense group's dwords.
__device__ __forceinline__ uint32_t idx_dword(const uint8_t *p, int dw, bool dense3) {
    const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
    if (!dense3) return q[dw];
    const uint32_t *g = q + 3 * (dw >> 2);
    const int w = dw & 3;
    if (w < 3) {
        const uint32_t x = g[w];
        return (d3_even(x) << 4) | d3_odd(x);
    }
    return d3_nibbles(g[0], g[1], g[2], 3);
}

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
// at LDS address m0 + l * size (m0 = wave-uniform destination).  The destination
// is an operand bound to m0 (the compiler writes m0); the s_nop is the one wait
// state an SALU write of m0 needs before a load with LDS = 1, which the compiler
// does not insert for an asm statement.
//   copy16:  16 bytes from the uniform base `src` + per-lane 32-bit offset.
//   copy16v: 16 bytes from a per-lane address.
//   copy4s:  4 bytes from the uniform base `src` + per-lane 32-bit offset.
//   copy4:   4 bytes from a per-lane address.
__device__ __forceinline__ void copy16(const uint8_t *src, uint32_t voff, uint32_t dst) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(src), "{m0}"(dst) : "memory");
}
__device__ __forceinline__ void copy16v(const uint8_t *src, uint32_t dst) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(dst) : "memory");
}
__device__ __forceinline__ void copy4s(const uint8_t *src, uint32_t voff, uint32_t dst) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(src), "{m0}"(dst) : "memory");
}
__device__ __forceinline__ void copy4(const uint8_t *src, uint32_t dst) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "{m0}"(dst) : "memory");
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
// The same for a wave-uniform int (kept in an SGPR): code that uses the result
// cannot be moved above the point where it is taken.
__device__ __forceinline__ int opaque_s(int x) {
    asm volatile("" : "+s"(x));
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
