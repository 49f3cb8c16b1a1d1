// Pieces shared by the attention kernels that keep a 64-key tile's V in LDS as
// fp16 V'^T rows (rq_prefill.hip, rq_attention.hip): the MFMA wrappers, the
// query rotation, the online-softmax + P V step of one tile and the epilogue.
//
// Layouts (wave64, lane l, g = l / 16, col = l % 16):
//   scores S^T (16 keys x 16 query positions per key block b): lane (g, col)
//     holds position col's scores of keys 16b + 4g + i, i = 0..3, b = 0..3;
//   O^T = V'^T P'^T on v_mfma_f32_16x16x32_f16 (A 16 x 32: lane holds row l % 16,
//     k = 8g .. 8g+7), two k-steps per tile: k-step s, element j of lane group g
//     is key 32s + 4g + j (j < 4) or 32s + 16 + 4g + j - 4 (j >= 4) -- exactly the
//     scores the lane holds, so P needs no transpose; acc[m] holds position col's
//     output dims 16m + 4g + i.
#pragma once

#include "rq_common.h"

namespace rq {

typedef __attribute__((ext_vector_type(4))) int i32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;

constexpr int kAttnD = 128;  // head_dim
constexpr int kAttnKT = 64;  // keys per tile
constexpr int kAttnPQ = 16;  // query positions per wave
constexpr float kAttnLog2e = 1.4426950408889634f;

// fp16 MFMA of the P V product (fp32 accumulation).
__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
}

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;

// 16-bit MFMA in the q dtype (bf16 or fp16 operands, fp32 accumulation): Q K^T
// over K rounded to the q dtype.
template <int DT>
__device__ __forceinline__ f32x4 mfma_qk(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (DT == RQ_DTYPE_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    else
        return mfma_f16(a, b, c);
}

// Two fp32 values rounded to fp16, packed low | high << 16 (one v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pack_f16(float lo, float hi) {
    typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
    const f16x2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// V'^T tile: 128 dim rows of 64 fp16 keys (128 bytes), 16-byte piece c of row d
// at d * 128 + 16 * (c ^ (d & 7)) (XOR swizzle: the 16 rows an MFMA operand read
// touches fall in distinct bank groups).  Key t = 16b + 4gg + i sits in piece
// 4 (b >> 1) + gg, element 4 (b & 1) + i.
__host__ __device__ constexpr int vt_piece(int d, int c) { return d * 128 + 16 * (c ^ (d & 7)); }

// 8 consecutive head dims base .. base+7 (base a multiple of 8) of q_rot = q R^T
// (xin: those dims of q; qr: the 8 results),
// each rounded to the q dtype: R is block diagonal with 2- or 4-wide blocks, so
// the 8 dims need only these 8 inputs.  Each output is the fma chain over its
// block in increasing k, starting from the first product
// (fused_paged_rq_decode.py:271 computes q.f32 @ R^T, then casts).
template <int DT>
__device__ __forceinline__ void rotate_q8(const float *xin, int base, const float *R, int rot_block, float *qr) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int j = base + k;
        float acc;
        if (rot_block == 4) {  // R[j][4 (j / 4) + i], i < 4
            const float4 r = *reinterpret_cast<const float4 *>(R + (int64_t)j * kAttnD + (j & ~3));
            const int b0 = k & ~3;
            acc = __builtin_fmaf(xin[b0], r.x, 0.f);
            acc = __builtin_fmaf(xin[b0 + 1], r.y, acc);
            acc = __builtin_fmaf(xin[b0 + 2], r.z, acc);
            acc = __builtin_fmaf(xin[b0 + 3], r.w, acc);
        } else {  // R[j][2 (j / 2) + i], i < 2
            const float2 r = *reinterpret_cast<const float2 *>(R + (int64_t)j * kAttnD + (j & ~1));
            const int b0 = k & ~1;
            acc = __builtin_fmaf(xin[b0], r.x, 0.f);
            acc = __builtin_fmaf(xin[b0 + 1], r.y, acc);
        }
        qr[k] = Elem<DT>::to_f32(Elem<DT>::from_f32(acc));
    }
}

// Work item of a workgroup in a grid (query blocks, kv heads, sequences).
// Workgroups are dispatched round-robin over the 8 XCDs, each with its own L2.
// Each (sequence, kv head) pair's query blocks are cut into S slices (S = 8 / kv
// heads when that divides both 8 and the query blocks, else 1), and the
// (pair, slice) units are dealt to the XCDs in order: XCD j takes units j, j + 8,
// ... one after another.  So the query blocks that stream one pair's keys share
// S L2s, and each sequence's work is spread over all 8 XCDs: with whole pairs
// (S = 1) and 4 kv heads, the XCDs 0-3 would hold the even and 4-7 the odd
// sequences, whatever their lengths.  Slice c of a pair holds its query blocks
// c, c + S, ... (causal blocks grow heavier with the position), and within a slice
// the last (heaviest) query blocks go first.  When the units do not divide into 8,
// the plain order.  Both are bijections of the grid onto (query block, kv head,
// sequence).
__device__ __forceinline__ void attn_work_item(int &qblk, int &h, int64_t &seq) {
    const uint32_t nx = gridDim.x, ny = gridDim.y;
    const uint32_t lin = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
    uint32_t pair = blockIdx.y + ny * blockIdx.z, xo = blockIdx.x;
    // S: 2, 4 or 8 (a power of two) for 4, 2 or 1 kv heads; 1 otherwise
    const uint32_t S = (ny == 1u || ny == 2u || ny == 4u) && nx % (8u / ny) == 0 ? 8u / ny : 1u;
    const uint32_t k = lin >> 3;  // rank of this workgroup on its XCD
    if (S == 1u) {
        if ((ny * gridDim.z) % 8u == 0) {
            pair = (lin & 7u) + 8u * (k / nx);
            xo = k % nx;
        }
    } else {  // 8 units per sequence: always a multiple of 8
        const uint32_t sh = __builtin_ctz(S);
        const uint32_t len = nx >> sh;                   // query blocks per slice
        const uint32_t u = (lin & 7u) + 8u * (k / len);  // (pair, slice) unit
        pair = u >> sh;
        xo = ((k % len) << sh) + (u & (S - 1u));  // slice c: query blocks c, c + S, ... (heavy and light mixed)
    }
    qblk = (int)(nx - 1 - xo);
    h = (int)(pair % ny);
    seq = pair / ny;
}

// Running state of one wave's 16 query positions (one per lane column).
// acc = sum P' V' and lsum = sum P' 2^-e_v carry the same factor 2^-e_run, so
// out = acc / l; m_run is in the score's base-2 units divided by sq.
struct AttnState {
    f32x4 acc[8];
    f32x4 lsum;  // row 0 (lanes g = 0, element 0): the row sum of the weights
    float m_run;
    int e_run;
    __device__ __forceinline__ void init() {
#pragma unroll
        for (int m = 0; m < 8; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
        lsum = f32x4{0.f, 0.f, 0.f, 0.f};
        m_run = -INFINITY;
        e_run = -14;
    }
};

// Row-sum operand of a tile: lanes of MFMA row 0 (col == 0) hold 2^-e_v in fp16
// (normal or denormal), the others zero.
__device__ __forceinline__ u32x4 rowsum_operand(int e_v, int col) {
    const uint32_t w = col == 0 ? pack_f16(ldexpf(1.f, -e_v), ldexpf(1.f, -e_v)) : 0u;
    return u32x4{w, w, w, w};
}

// Online softmax over one tile and O^T += V'^T P'^T.
//   s: this lane's 16 scores (masked ones -INFINITY); the base-2 score proper is
//      s * s_unit * sq (s_unit: per tile, sq: per position);
//   e_v: the tile's V exponent, V' = V 2^-e_v in fp16 (|V'| below max|centroid|);
//   vt: the tile's V'^T rows; koff0 / koff1: this lane's pieces g and 4 + g of row
//       col (vt_piece(col, g), vt_piece(col, 4 + g));
//   ones: the tile's row-sum operand (rowsum_operand(e_v, col), col = lane % 16).
__device__ __forceinline__ void softmax_pv(AttnState &st, const float (&s)[16], float s_unit, float sq, int e_v,
                                           const uint8_t *vt, int koff0, int koff1, const u32x4 ones) {
    float tmax = s[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) tmax = fmaxf(tmax, s[i]);
    tmax = rows_max(tmax) * s_unit;
    // Lazy running max: rescale only when a position's max exceeds m_run by more
    // than 8 in log2 units, so p <= 2^8 in between (P' = p 2^(e_v - e_run) <= 2^8
    // stays in fp16); acc and lsum are relative to the same m_run either way.
    if (__any((tmax - st.m_run) * sq > 8.f)) {
        const float m_new = fmaxf(st.m_run, tmax);
        const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f((st.m_run - m_new) * sq);
#pragma unroll
        for (int m = 0; m < 8; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) st.acc[m][i] *= alpha;
        st.lsum *= alpha;
        st.m_run = m_new;
    }
    // V exponent of the tile: acc carries 2^-e_run, and P' = p 2^(e_v - e_run) <= 2^8
    // in fp16 (the exponent's fma adds e_v - e_run).  The row sum is one more MFMA
    // row: sum P' 2^-e_v = 2^-e_run sum p, with the same rounded weights as the
    // numerator (the reference sums p in fp32 and rounds it for P V,
    // fused_paged_rq_int8_prefill.py:214-229).
    if (e_v > st.e_run) {  // uniform: one tile per workgroup
        const float f = ldexpf(1.f, st.e_run - e_v);
#pragma unroll
        for (int m = 0; m < 8; ++m) st.acc[m] *= f;
        st.lsum *= f;
        st.e_run = e_v;
    }
    const float bias = (st.m_run == -INFINITY ? 0.f : -st.m_run * sq) + (float)(e_v - st.e_run);
    const float usq = s_unit * sq;
    // k-step t takes the scores of key blocks 2t and 2t + 1, in the lane's order.
    u32x4 pop[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * t + e], usq, bias));
        pop[t] = u32x4{pack_f16(p[0], p[1]), pack_f16(p[2], p[3]), pack_f16(p[4], p[5]), pack_f16(p[6], p[7])};
    }
    st.lsum = mfma_f16(ones, pop[0], st.lsum);
    st.lsum = mfma_f16(ones, pop[1], st.lsum);
    // 8 blocks of 16 head dims (dim 16m + col; its swizzle term is col & 7), two k-steps
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const u32x4 v0 = *reinterpret_cast<const u32x4 *>(vt + 16 * m * 128 + koff0);
        const u32x4 v1 = *reinterpret_cast<const u32x4 *>(vt + 16 * m * 128 + koff1);
        st.acc[m] = mfma_f16(v0, pop[0], st.acc[m]);
        st.acc[m] = mfma_f16(v1, pop[1], st.acc[m]);
    }
}

// 1 / (row sum of the weights) of this lane's position (0 when nothing was seen).
__device__ __forceinline__ float attn_inv_l(const AttnState &st) {
    const float l_run = rows_sum(st.lsum[0]);  // rows 4g: only g = 0 holds row 0
    return l_run > 0.f ? 1.f / l_run : 0.f;
}

// Epilogue of one position (lane column): out_rot = acc / l rounded to the q
// dtype, rotated back by R and rounded again.  Lane (g, col) holds dims
// 16m + 4g + i (i = 0..3): a whole 4-dim block of R (or two 2-dim ones, whose
// off-block entries are exact zeros), so the back-rotation runs in registers:
// out[d] = fma chain over the block in increasing k of round(o[k]) * R[k][d]
// (fused_paged_rq_decode.py:308 order).  g = lane / 16.
template <int DT>
__device__ __forceinline__ void store_rotated(const AttnState &st, float inv_l, uint16_t *orow, const float *R,
                                              int rot_block, int g) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int d0 = 16 * m + 4 * g;
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = Elem<DT>::to_f32(Elem<DT>::from_f32(st.acc[m][i] * inv_l));
        float4 r[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = *reinterpret_cast<const float4 *>(R + (int64_t)(d0 + i) * kAttnD + d0);
        const float rc[4][4] = {{r[0].x, r[0].y, r[0].z, r[0].w}, {r[1].x, r[1].y, r[1].z, r[1].w},
                                {r[2].x, r[2].y, r[2].z, r[2].w}, {r[3].x, r[3].y, r[3].z, r[3].w}};
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v;
            if (rot_block == 4) {
                v = o[0] * rc[0][j];
                v = __builtin_fmaf(o[1], rc[1][j], v);
                v = __builtin_fmaf(o[2], rc[2][j], v);
                v = __builtin_fmaf(o[3], rc[3][j], v);
            } else {
                const int k0 = j & 2;  // first row of d0 + j's 2-dim block
                v = o[k0] * rc[k0][j];
                v = __builtin_fmaf(o[k0 + 1], rc[k0 + 1][j], v);
            }
            w[j] = Elem<DT>::from_f32(v);
        }
        *reinterpret_cast<uint2 *>(orow + d0) = make_uint2(w[0] | (w[1] << 16), w[2] | (w[3] << 16));
    }
}

}  // namespace rq
