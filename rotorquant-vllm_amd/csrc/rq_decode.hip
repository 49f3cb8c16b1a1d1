// Fused paged decode attention over the packed RotorQuant cache (gfx950).
//
// Replaces fused_paged_rq_decode (src/rotorquant_vllm/triton/fused_paged_rq_decode.py:214-312,
// kernel :32-206).  Same mathematics -- attention in the rotated space with
// q_rot = dtype(q R^T) (:271), K = dtype(centroid[idx] * norm) (:146-147) and V
// likewise (:190-191), exp2 online softmax, out = dtype(dtype(out_rot) R) (:201-206,
// :308) -- organised for CDNA4 in three launches:
//
//   * decode_prep_kernel: per sequence, the Q^T MFMA operand (q_rot in the q dtype)
//     of every kv head and one descriptor per 32-token tile (slot offsets from the
//     block table);
//   * decode_kernel: persistent; the tiles of the whole batch are split into
//     contiguous ranges, one per resident workgroup.  A workgroup holds one wave
//     per kv head, so each token's K/V bytes are read once and shared by all GQA
//     query heads.  Tiles are copied global -> LDS two ahead.  Per tile, each lane
//     builds half of one token's K and V codebook tables -- the 8 (16) values
//     dtype(c_j * norm) of that token -- in LDS; the lanes holding the token's
//     indices look them up with v_perm_b32.  Q K^T runs on the q-dtype MFMA (exact
//     products, fp32 sums), P V on the fp16 MFMA with V as an fp16 image of its
//     q-dtype value.  Each sequence segment of a range ends in an (m, l, acc)
//     partial;
//   * decode_merge_kernel: log-sum-exp over a sequence's partials, rounding and
//     the rotation back by R.
//
// MFMA operand layout used below (16x16x32, wave64, lane l, g = l / 16):
//   A (16 x 32): lane holds row l % 16, k = 8g .. 8g+7   (4 dwords of 2 x 16-bit)
//   B (32 x 16): lane holds col l % 16, k = 8g .. 8g+7
//   C (16 x 16): lane holds col l % 16, rows 4g .. 4g+3  (4 floats)
//
// S^T = K Q^T per 16-token group j (A = K: row = token 16j + l%16, k = head dims;
// B = Q^T: col = query head).  Lane (g, col) then holds the scores of tokens
// 4g + i (j = 0) and 16 + 4g + i (j = 1) for its query head.
// O^T = V^T P^T with one row per *pair* of head dims of a nibble dword (row r:
// dims 8r .. 8r+7, pairs (e0,e2) (e1,e3) (e4,e6) (e5,e7) in four MFMAs): k slots
// 8g + 2i and 8g + 2i + 1 hold the two dims of the pair for token 16kb + 4g + i,
// so a lane's V operand is one token's table lookups (no transpose), and the P^T
// column picks the dim.  With at most 8 query heads per kv head, columns c < 8
// carry (p, 0) for head c and columns c >= 8 carry (0, p) for head c - 8 (the S^T
// columns repeat the heads likewise): one MFMA yields both dims of the pair.
// With more heads (WIDE), two MFMAs per pair, (p, 0) and (0, p).
#include <algorithm>
#include <mutex>
#include <type_traits>

#include <hip/hip_ext.h>

#include "rq_common.h"

namespace rq {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;

constexpr int kD = 128;          // head_dim handled by this kernel
constexpr int kTile = 32;        // tokens per inner iteration
constexpr int kMaxWaves = 8;     // kv heads (= waves) per workgroup
constexpr int kMaxKvHeads = 64;
constexpr float kLog2e = 1.4426950408889634f;

template <int DT>
__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (DT == RQ_DTYPE_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
}

// Two fp32 values rounded to the 16-bit dtype, packed a | b << 16 (one
// v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32).
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    typedef __attribute__((ext_vector_type(2))) float f32x2;
    if constexpr (DT == RQ_DTYPE_BF16) {
        typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
    } else {
        typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
    }
}

// One packed dword (8 nibbles, coordinates e0..e7 of one token) -> MFMA
// operand of 8 16-bit values in the order e0 e2 e4 e6 e1 e3 e5 e7.
template <int BITS>
__device__ __forceinline__ u32x4 decode_row8_sel(const Table16 &t, uint32_t even, uint32_t odd) {
    uint2 e = lookup4<BITS>(t, even), o = lookup4<BITS>(t, odd);
    return u32x4{e.x, e.y, o.x, o.y};
}
template <int BITS>
__device__ __forceinline__ u32x4 decode_row8(const Table16 &t, uint32_t x) {
    return decode_row8_sel<BITS>(t, (x >> 4) & 0x0f0f0f0fu, x & 0x0f0f0f0fu);  // e0 e2 e4 e6 | e1 e3 e5 e7
}

// ---------------------------------------------------------------------------
// Per-token codebook tables in LDS.  A table holds the 16-bit values of a
// token's 2^BITS codebook entries as low-byte / high-byte dwords (Table16):
//   8 entries  (16 bytes): lo0 hi0 lo1 hi1          (lo0: low bytes of entries 0-3)
//   16 entries (32 bytes): lo0 hi0 lo1 hi1 lo2 hi2 lo3 hi3
// Half hh (entries [NE/2 hh, NE/2 (hh + 1))) is written by one lane: 8 bytes at
// 8 hh of the first 16-byte piece, or the 16-byte piece hh (the two pieces of a
// 32-byte table need not be adjacent).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint2 planes4(uint32_t p01, uint32_t p23) {  // 4 values as pairs -> (lo, hi) dwords
    return make_uint2(perm(p23, p01, 0x06040200u), perm(p23, p01, 0x07050301u));
}

// Half hh of the table of dtype(c_j * m) for the codebook cb (16 floats in LDS,
// zero-padded), written at dst.  F16_IMAGE: the values are then stored as fp16
// (for a bf16 dtype: the bf16 value converted to fp16, exact while it is at least
// 2^-17 and below 65504).  The product is rounded to fp32 before the 16-bit
// rounding, as the reference's fp32 multiply followed by .to(dtype).
template <int DT, int BITS, bool F16_IMAGE>
__device__ __forceinline__ void table_half(const float *cb, float m, int hh, uint8_t *dst0, uint8_t *dst1) {
    constexpr int NH = (1 << BITS) / 2;  // entries per half
    const float4 *c4 = reinterpret_cast<const float4 *>(cb + NH * hh);
    uint32_t pr[NH / 2];
#pragma unroll
    for (int q = 0; q < NH / 4; ++q) {
        const float4 c = c4[q];
        const float e[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            uint32_t v = pack2<DT>(opaque(e[2 * j] * m), opaque(e[2 * j + 1] * m));
            if constexpr (F16_IMAGE && DT == RQ_DTYPE_BF16)
                v = pack2<RQ_DTYPE_F16>(__uint_as_float(v << 16), __uint_as_float(v & 0xffff0000u));
            pr[2 * q + j] = v;
        }
    }
    if constexpr (NH == 4) {
        *reinterpret_cast<uint2 *>(dst0 + 8 * hh) = planes4(pr[0], pr[1]);
    } else {
        const uint2 x = planes4(pr[0], pr[1]), y = planes4(pr[2], pr[3]);
        *reinterpret_cast<u32x4 *>(hh ? dst1 : dst0) = u32x4{x.x, x.y, y.x, y.y};
    }
}

template <int BITS>
__device__ __forceinline__ Table16 read_table(const uint8_t *p0, const uint8_t *p1) {
    Table16 t;
    const u32x4 r = *reinterpret_cast<const u32x4 *>(p0);
    t.lo[0] = r.x, t.hi[0] = r.y, t.lo[1] = r.z, t.hi[1] = r.w;
    if constexpr (BITS == 4) {
        const u32x4 s = *reinterpret_cast<const u32x4 *>(p1);
        t.lo[2] = s.x, t.hi[2] = s.y, t.lo[3] = s.z, t.hi[3] = s.w;
    } else {
        t.lo[2] = t.lo[3] = t.hi[2] = t.hi[3] = 0u;
    }
    return t;
}

// Value of lane (l & ~3) + perm[l & 3] of the lane's quad (DPP quad_perm, ctrl =
// perm[0] | perm[1] << 2 | perm[2] << 4 | perm[3] << 6).
template <int CTRL>
__device__ __forceinline__ uint32_t quad_pick(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xf, 0xf, false);
}

struct TileDesc;

struct DecodeArgs {
    const void *q;
    int64_t q_ss, q_sh;
    const uint8_t *cache;
    int64_t stride_block, stride_token;
    int block_size;
    int bs_shift;       // log2(block_size), or -1 when block_size is not a power of two
    int H, G, HQ;
    const int32_t *bt;
    int64_t bt_ss;
    int64_t max_blocks;
    const int32_t *seq_lens;
    const float *kc, *vc;
    int nkc, nvc;
    const float *R;
    int rot_block;
    float score_scale;  // sm_scale * log2(e)
    int max_len;        // min(max_blocks * block_size, max_seq_len): lengths are clamped to it
    int64_t num_blocks; // physical blocks; table entries outside [0, num_blocks) read block 0
    int hpw;            // kv heads per workgroup = waves per workgroup (divides H, <= 8)
    int tok_stride;     // LDS bytes per staged token: 2 * index bytes * hpw (K and V indices) + 16 (bank skew)
    int stage_bytes;    // LDS bytes per stage: kTile * tok_stride + 2 * hpw * kTile * 4 (norms)
    int grid_w;         // decode workgroups per kv-head group (the tile ranges)
    int split_c;        // workgroups per rank: workgroup w has rank min(w / split_c, 3)
    int wt[4];          // tile weight of a workgroup of each rank
    uint64_t split_r;   // floor((2^64 - 1) / total weight)
    TileDesc *descs;    // [total tiles] (prep kernel)
    int *tile_prefix;   // [seq][2]: first workgroup whose range covers the sequence, number of such workgroups
    int *n_tiles_total;
    uint64_t *split_m;  // M of the range split (prep kernel)
    uint32_t *qops;     // [seq][H][16 cols][4 g][4 chunks][4 dwords]: q-dtype query operands (cols < G written)
    float *part_acc;    // [slot][HQ][D], slot = workgroup + seq
    float *part_ml;     // [slot][HQ][2]
    void *out;
    int64_t o_ss, o_sh;
};

// The lane index, recomputed where it is used (two VALU ops, no input register).
// Lane-derived values needed only at segment boundaries or by the copy issue are
// built from it: the register allocator otherwise keeps them live across the tile
// loop and, under pressure, spills them, and a spill reload inside the loop is a
// vector-memory load whose wait also waits for every copy in flight.
__device__ __forceinline__ uint32_t lane_now() {
    uint32_t x;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(x));
    return x;
}

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, l);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), l);
    return ((uint64_t)hi << 32) | lo;
}

// q_rot = q R^T of the G query heads of (seq, kv head h), rounded to the query
// dtype (fused_paged_rq_decode.py:271), as the Q^T MFMA operand in that dtype:
// lane (g, col) holds for dim chunk c the dims 32g + 8c + {0,2,4,6,1,3,5,7} of
// query head col (zero for col >= G).
// wq: this wave's LDS scratch of G * 128 16-bit values.
template <int DT>
__device__ __forceinline__ void query_operand(const DecodeArgs &a, int64_t seq, int h, uint16_t *wq, u32x4 (&qop)[4]) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, col = lane & 15;
    {
        // Lane: dims j, j+1 (one rotation block; rb is 2 or 4).  The q loads of four
        // query heads are issued together.
        const int rb = a.rot_block;
        const int j = 2 * lane;
        const int k0 = (j / rb) * rb;
        float r0[4], r1[4];
        if (rb == 4) {
            const float4 x = *reinterpret_cast<const float4 *>(a.R + j * kD + k0);
            const float4 y = *reinterpret_cast<const float4 *>(a.R + (j + 1) * kD + k0);
            r0[0] = x.x, r0[1] = x.y, r0[2] = x.z, r0[3] = x.w;
            r1[0] = y.x, r1[1] = y.y, r1[2] = y.z, r1[3] = y.w;
        } else {
            const float2 x = *reinterpret_cast<const float2 *>(a.R + j * kD + k0);
            const float2 y = *reinterpret_cast<const float2 *>(a.R + (j + 1) * kD + k0);
            r0[0] = x.x, r0[1] = x.y, r0[2] = 0.f, r0[3] = 0.f;
            r1[0] = y.x, r1[1] = y.y, r1[2] = 0.f, r1[3] = 0.f;
        }
        const uint16_t *qbase = reinterpret_cast<const uint16_t *>(a.q) + seq * a.q_ss + (int64_t)(h * a.G) * a.q_sh + k0;
        for (int qh0 = 0; qh0 < a.G; qh0 += 4) {
            uint2 raw[4];
    #pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint16_t *qp = qbase + (int64_t)min(qh0 + u, a.G - 1) * a.q_sh;
                raw[u] = rb == 4 ? *reinterpret_cast<const uint2 *>(qp) : make_uint2(*reinterpret_cast<const uint32_t *>(qp), 0u);
            }
    #pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t w4[2] = {raw[u].x, raw[u].y};
                float acc0 = 0.f, acc1 = 0.f;
    #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (i < rb) {
                        const float x = Elem<DT>::to_f32((w4[i >> 1] >> (16 * (i & 1))) & 0xffffu);
                        acc0 = __builtin_fmaf(x, r0[i], acc0);
                        acc1 = __builtin_fmaf(x, r1[i], acc1);
                    }
                }
                if (qh0 + u < a.G)
                    reinterpret_cast<uint32_t *>(wq + (qh0 + u) * kD)[lane] =
                        Elem<DT>::from_f32(acc0) | (Elem<DT>::from_f32(acc1) << 16);
            }
        }
    }
    __builtin_amdgcn_wave_barrier();
    #pragma unroll
    for (int c = 0; c < 4; ++c) {
        // w: dims 8c' .. 8c'+7 (c' = 4g + c) as 16-bit pairs (d0 d1) (d2 d3) (d4 d5) (d6 d7)
        const uint4 w = col < a.G ? *reinterpret_cast<const uint4 *>(wq + col * kD + 32 * g + 8 * c)
                                  : make_uint4(0, 0, 0, 0);
        qop[c] = u32x4{perm(w.y, w.x, 0x05040100u), perm(w.w, w.z, 0x05040100u),   // (d0 d2) (d4 d6)
                       perm(w.y, w.x, 0x07060302u), perm(w.w, w.z, 0x07060302u)};  // (d1 d3) (d5 d7)
    }
    __builtin_amdgcn_wave_barrier();
}

// s_waitcnt vmcnt(min(n, HI)) for a wave-uniform n >= LO (binary search over the
// immediates; a count above HI waits for more than needed, never for less).
template <int LO, int HI>
__device__ __forceinline__ void wait_copies_upto(int n) {
    if constexpr (LO >= HI) {
        wait_copies<HI>();
    } else {
        constexpr int MID = (LO + HI + 1) / 2;
        if (n >= MID) wait_copies_upto<MID, HI>(n);
        else wait_copies_upto<LO, MID - 1>(n);
    }
}

// Tile descriptor: one 32-token tile of one sequence, written by the prep kernel
// and read by the decode workgroup that owns the tile.
struct TileDesc {
    int32_t seq, tile, valid, pad;  // sequence, tile index inside it, tokens in the tile (1..32)
    uint64_t off[kTile];            // byte offset of each token's slot (0 past `valid`)
};
static_assert(sizeof(TileDesc) == 16 + 8 * kTile, "TileDesc layout");
constexpr int kDescPieces = (int)sizeof(TileDesc) / 16;  // 16-byte copy pieces per descriptor

// Pipeline depth of a decode variant (hpw kv heads per workgroup, dense layout d3):
// NS stages, tile t + NS copied into the stage of tile t once it is consumed.  The
// descriptor ring holds at least twice as many descriptors as there are stages: the
// descriptor of tile t + NS is then copied before the copies of tile t, so the wait
// for tile t covers it (and the descriptors of tiles t+1 .. t+2 read for the query
// look-ahead).  Two stages everywhere: deeper pipelines for the small stages of one
// or two heads per workgroup were measured slower (six stages at one head: the
// initial copies of all workgroups, 26 MB at once, delayed every first tile by
// ~4 us, and the loop itself is bound by one wave's latency per SIMD, not copies).
constexpr bool decode_line_copies(int hpw, bool d3) { return (hpw == 1 || hpw == 2) && !d3; }
constexpr int decode_stages(int hpw, bool d3) { return (void)hpw, (void)d3, 2; }
constexpr int decode_ring(int hpw, bool d3) { return decode_stages(hpw, d3) == 2 ? 4 : decode_stages(hpw, d3) <= 4 ? 8 : 16; }
static_assert(decode_ring(1, false) >= 2 * decode_stages(1, false) && decode_ring(2, false) >= 2 * decode_stages(2, false) &&
                  decode_ring(8, false) >= 2 * decode_stages(8, false),
              "descriptor ring too small for the stages");

// First tile of workgroup w's range, w in [0, grid_w]: the tiles of all
// sequences are split into contiguous ranges by weight.  With several workgroups
// per CU, the ones dispatched first onto each CU (rank 0: w < split_c, one per CU)
// are favoured by the wave arbiter and run well ahead of the later ones
// (measured: with equal ranges and two per CU, rank 0 ends at ~0.7x the other's
// time); weighting the ranks (65:35 for two per CU, the best of a sweep) shortens
// the tail in which CU slots idle.
// The split is s(w) * M >> 32 with M ~ NT 2^32 / s(grid_w) (M = the high half of
// (NT << 32) * split_r, at most the exact quotient), computed once by the prep
// kernel; the decode and the merge kernel evaluate exactly this, and the last
// range ends at NT.
struct RangeSplit {
    int c, G, NT;
    int w0, w1, w2, w3;  // rank weights
    uint64_t M;
};
__device__ __forceinline__ uint64_t split_multiplier(const DecodeArgs &a, int NT) {
    return __umul64hi((uint64_t)NT << 32, a.split_r);
}
__device__ __forceinline__ RangeSplit make_split(const DecodeArgs &a, int NT) {
    return RangeSplit{a.split_c, a.grid_w, NT, a.wt[0], a.wt[1], a.wt[2], a.wt[3], *a.split_m};
}
// r by value: through a reference the rank select below is turned into an indexed
// load of the struct, which the compiler then moves to LDS.
__device__ __forceinline__ int range_start(const RangeSplit r, int w) {
    if (w >= r.G) return r.NT;
    const int rank = min(w / r.c, 3);
    const int wr = rank == 0 ? r.w0 : rank == 1 ? r.w1 : rank == 2 ? r.w2 : r.w3;
    uint64_t s = (uint64_t)(w - rank * r.c) * wr;
    if (rank > 0) s += (uint64_t)r.c * r.w0;
    if (rank > 1) s += (uint64_t)r.c * r.w1;
    if (rank > 2) s += (uint64_t)r.c * r.w2;
    return (int)((s * r.M) >> 32);
}


__device__ __forceinline__ int seq_tiles(const DecodeArgs &a, int64_t b) {
    const int L = min(a.seq_lens[b], a.max_len);
    return L > 0 ? (L + kTile - 1) / kTile : 0;
}

// Per-call preparation; workgroup (seq, y):
//   * y == 0: the query operands of every kv head of the sequence, stored per
//     query-head column (256 bytes each, in the order the decode lanes (g, col)
//     read them) so one copy moves a kv head's G columns;
//   * y >= 1: the tile descriptors of the sequence's tokens, four per thread and
//     step, placed after the tiles of the sequences before it (the tiles of all
//     sequences, in order, form the work the decode kernel splits by range);
//   * tile_prefix[seq] = the first decode workgroup whose range covers the
//     sequence and the number of such workgroups (for the merge); the last
//     sequence also stores the total tile count and the range-split multiplier.
template <int DT>
__global__ __launch_bounds__(512) void decode_prep_kernel(DecodeArgs a) {
    const int64_t seq = blockIdx.x;
    const int y = blockIdx.y;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int nw = blockDim.x >> 6;
    extern __shared__ __align__(16) uint8_t prep_lds[];  // query staging, 16 x kD 16-bit values per wave
    __shared__ int part[2 * kMaxWaves];
    // a descriptor workgroup past the end of its sequence's tokens has nothing to do
    if (y >= 1 && 4 * (y - 1) * (int)blockDim.x >= seq_tiles(a, seq) * kTile) return;
    if (y == 0) {
        for (int h = wave; h < a.H; h += nw) {
            u32x4 qop[4];
            query_operand<DT>(a, seq, h, reinterpret_cast<uint16_t *>(prep_lds) + wave * 16 * kD, qop);
            const int g = lane >> 4, col = lane & 15;
            uint4 *dst = reinterpret_cast<uint4 *>(a.qops + ((seq * a.H + h) * 16 + col) * 64 + g * 16);
            if (col < a.G) {
    #pragma unroll
                for (int c = 0; c < 4; ++c) dst[c] = make_uint4(qop[c].x, qop[c].y, qop[c].z, qop[c].w);
            }
        }
    }
    // tiles before this sequence (prefix) and in all sequences (NT)
    int cnt = 0, tot = 0;
    for (int64_t b = threadIdx.x; b < gridDim.x; b += blockDim.x) {
        const int nb = seq_tiles(a, b);
        cnt += b < seq ? nb : 0;
        tot += nb;
    }
    for (int o = 32; o >= 1; o >>= 1) {
        cnt += __shfl_xor(cnt, o);
        tot += __shfl_xor(tot, o);
    }
    if (lane == 0) {
        part[wave] = cnt;
        part[kMaxWaves + wave] = tot;
    }
    __syncthreads();
    int prefix = 0, NT = 0;
    for (int w = 0; w < nw; ++w) {
        prefix += part[w];
        NT += part[kMaxWaves + w];
    }
    const int n = seq_tiles(a, seq);
    const int L = min(a.seq_lens[seq], a.max_len);
    if (y == 0 && wave == 0) {
        // The decode workgroups whose ranges cover this sequence (for the merge):
        // the owner of tile t is the number of w in [1, G) with range_start(w) <= t
        // (range_start is non-decreasing and range_start(0) = 0).
        const RangeSplit r{a.split_c, a.grid_w, NT, a.wt[0], a.wt[1], a.wt[2], a.wt[3], split_multiplier(a, NT)};
        // c(t) = #{w in [1, G): range_start(w) <= t}, in two rounds of 64 evaluations:
        // lane k tests w = 1 + k * step (a ballot brackets the answer), then w = 1 + base
        // + k within the bracket (step <= 64 while G <= 4097; beyond that a lane loop).
        const int step = (r.G - 1 + 63) / 64;
        auto count_le = [&](int tk) {
            const int w1 = 1 + lane * step;
            const uint64_t m1 = __ballot(w1 < r.G && range_start(r, w1) <= tk);
            const int k = m1 ? 63 - __clzll(m1) : -1;  // last coarse point at or below tk
            if (k < 0) return 0;
            int c = k * step + 1;  // w = 1 .. 1 + k * step all count
            for (int j0 = 1; j0 < step; j0 += 64) {
                const int w2 = 1 + k * step + j0 + lane;
                const uint64_t m2 = __ballot(j0 + lane < step && w2 < r.G && range_start(r, w2) <= tk);
                c += __popcll(m2);
            }
            return c;
        };
        const int c_lo = count_le(prefix), c_hi = count_le(prefix + n - 1);
        if (lane == 0) {
            a.tile_prefix[2 * seq] = n > 0 ? c_lo : 0;
            a.tile_prefix[2 * seq + 1] = n > 0 ? c_hi - c_lo + 1 : 0;
            if (seq == gridDim.x - 1) {
                *a.n_tiles_total = NT;
                *a.split_m = r.M;
            }
        }
    }
    if (y == 0) return;  // the query operands above are this workgroup's share
    const int32_t *bt_row = a.bt + seq * a.bt_ss;
    // four consecutive tokens per thread and step (block-table loads issued together),
    // on the workgroups y = 1 .. gridDim.y - 1
    const int ny = gridDim.y - 1;
    for (int j0 = 4 * ((y - 1) * (int)blockDim.x + (int)threadIdx.x); j0 < n * kTile; j0 += 4 * ny * blockDim.x) {
        int phys[4];
    #pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int pos = j0 + u;
            const int lb = a.bs_shift >= 0 ? pos >> a.bs_shift : pos / a.block_size;
            phys[u] = pos < L ? bt_row[lb] : 0;
        }
        TileDesc *d = a.descs + prefix + j0 / kTile;
        uint64_t off[4];
    #pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int pos = j0 + u;
            const int in_blk = a.bs_shift >= 0 ? (pos & (a.block_size - 1)) : pos % a.block_size;
            const int64_t p = (phys[u] < 0 || phys[u] >= a.num_blocks) ? 0 : phys[u];
            off[u] = pos < L ? (uint64_t)(p * a.stride_block + (int64_t)in_blk * a.stride_token) : 0;
        }
        uint4 *o4 = reinterpret_cast<uint4 *>(&d->off[j0 % kTile]);
        o4[0] = make_uint4((uint32_t)off[0], (uint32_t)(off[0] >> 32), (uint32_t)off[1], (uint32_t)(off[1] >> 32));
        o4[1] = make_uint4((uint32_t)off[2], (uint32_t)(off[2] >> 32), (uint32_t)off[3], (uint32_t)(off[3] >> 32));
        if (j0 % kTile == 0) {
            d->seq = (int32_t)seq;
            d->tile = j0 / kTile;
            d->valid = min(kTile, L - j0);
            d->pad = 0;
        }
    }
}

// Decode.  The tiles of all sequences, in order, are split into contiguous ranges
// (see RangeSplit); workgroup w (with blockIdx.z selecting a group of hpw kv heads,
// one wave per head) takes range w, so every workgroup gets about the same work
// whatever the sequence lengths.  A range covers one or more sequence segments;
// each segment ends in a partial (m, l, acc) at slot w + seq, which is unique
// because ranges are contiguous and ordered.
//
// Data movement: tile descriptors are copied into an LDS ring of RING slots,
// RING tiles ahead, and each tile's K/V index runs and norms NS tiles ahead into
// NS stages (decode_stages: 2, or 3 / 6 for two / one kv heads per workgroup):
//   stage layout: token t at t * tok_stride: [K idx of the hpw heads | V idx]
//                 then the norms (2 * hpw x 32 fp32).
// One copy instruction moves a whole token's K+V index run (8*hpw x 16 B), so
// every request covers whole cache lines.  Iteration t: wait for tile t (tiles
// t+1 .. t+NS-1 stay in flight), barrier, read this wave's index bytes and
// norms, build the codebook tables into the wave's own K index bytes (read
// already), read the tables and look the V operands up, barrier, copy
// descriptor t+RING and tile t+NS, compute tile t from registers.  Each wave
// counts the copies it issues (every copy instruction has its first lane active,
// so none is skipped); the wait for tile t lets exactly the copies issued after
// tile t's stay in flight -- and none after the query operand of a segment that
// starts at tile t.
// Occupancy 4 (128 VGPRs) where the compiler fits the kernel without spilling.  One-
// and two-head workgroups (at most 8 and 4 per CU) put at most two waves on a SIMD,
// so they take 2 (256 VGPRs): at 4 their 4-bit variants spilled 20-116 bytes per lane
// into the loop.
constexpr int decode_waves_per_eu(int kb, int vb, int hpw) {
    return hpw == 1 || hpw == 2 ? 2 : (kb + vb == 6 || (kb + vb == 7 && hpw != 4)) ? 4 : 1;
}

// D3: the cache holds the dense 3-bit index layout (48 index bytes per head).
// WIDE: more than 8 query heads per kv head.
template <int DT, int KB, int VB, int HPW, bool D3, bool WIDE>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(decode_waves_per_eu(KB, VB, HPW)))) void decode_kernel(DecodeArgs a) {
    const int w = blockIdx.x;
    const int NT = *a.n_tiles_total;
    const RangeSplit rsp = make_split(a, NT);
    const int k0 = range_start(rsp, w);
    const int nt = range_start(rsp, w + 1) - k0;
    if (nt <= 0) return;

    // HPW > 0: heads per workgroup fixed at compile time (LDS offsets become immediates)
    const int hpw = HPW > 0 ? HPW : a.hpw;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & 63;
    const int h0 = blockIdx.z * hpw;
    const SlotLayout SL(a.H, kD, D3);
    constexpr int IB = D3 ? 48 : 64;   // index bytes per head
    constexpr bool kScaleV = DT == RQ_DTYPE_BF16;  // V fp16 image carries 2^-e_run (bf16 range)
    // One or two kv heads per workgroup (tensor-parallel slices): a token's K and V index
    // runs are only 128 * HPW bytes, so copies use all 64 lanes with per-lane addresses
    // (8 / HPW tokens per instruction) into tokens of 128 * HPW bytes whose 16-byte
    // pieces are XOR-swizzled (piece p of token t at 16 (p ^ swz(t))), which keeps the
    // operand reads free of bank conflicts.  Otherwise one instruction per token and a
    // 16-byte skew per token.
    constexpr bool kLine = decode_line_copies(HPW, D3);
    constexpr int NS = decode_stages(HPW, D3), RING = decode_ring(HPW, D3);
    const int TS = kLine ? 128 * HPW : (HPW > 0 ? 2 * IB * HPW + 16 : a.tok_stride);
    const int norm_off = kTile * TS;
    const int stage_bytes = HPW > 0 ? kTile * TS + 2 * HPW * kTile * 4 : a.stage_bytes;
    const int tl_copy = lane & 31;  // token of this lane's norm copy (rows layout)

    extern __shared__ __align__(16) uint8_t lds[];
    const TileDesc *const ring = reinterpret_cast<const TileDesc *>(lds + NS * stage_bytes);
    // Query operand slot: per wave, its kv head's G columns (256 bytes each); then
    // the K and V codebooks (16 floats each, zero-padded).
    const int G = a.G;
    uint8_t *const qarea = lds + NS * stage_bytes + RING * sizeof(TileDesc);
    float *const cbarea = reinterpret_cast<float *>(qarea + hpw * G * 256);

    // Byte offset in a stage of byte b of 16-byte piece p of token t (pieces: K indices
    // of the hpw heads, 4 per head, then V indices; nibble layouts).  swz(t) = (t >> 1) & 7
    // gives the 8 even (odd) tokens of 16 consecutive ones distinct pieces, and is equal
    // for tokens t, t + 1 and t + 16, so most operand addresses differ by immediates.
    auto swz = [](int t) { return (t >> 1) & 7; };
    auto at = [&](int t, int p, int b) { return t * TS + 16 * (kLine ? (p ^ swz(t)) : p) + b; };

    // Descriptor of local tile i -> ring slot i % RING (wave 0, one copy).  Each
    // issue function returns the number of copy instructions this wave issued.
    auto issue_desc = [&](int i) {
        const uint32_t l = lane_now();  // rebuilt here, not kept live across the loop
        if (wave == 0 && l < (uint32_t)kDescPieces)
            copy16(reinterpret_cast<const uint8_t *>(a.descs + k0 + i), 16 * l, lds_addr(reinterpret_cast<const uint8_t *>(ring + (i & (RING - 1)))));
        return wave == 0 ? 1 : 0;
    };
    // Copies of local tile i into stage sb.  Per wave and full tile: kTile / hpw
    // token copies (line copies: four) and one norm copy (HPW >= 4: on waves < hpw / 4).
    auto issue = [&](int i, const uint8_t *sb) {
        const TileDesc &d = ring[i & (RING - 1)];
        const int valid = __builtin_amdgcn_readfirstlane(d.valid);
        int n = 0;
        const uint64_t base = d.off[lane_now() & 31];
        const uint32_t dst = lds_addr(sb);
        constexpr int PH = IB / 16;  // 16-byte pieces per head
        const uint32_t kv_src = lane < PH * hpw ? (uint32_t)(SL.k_idx + IB * h0 + 16 * lane)
                                                : (uint32_t)(SL.v_idx + IB * h0 + 16 * (lane - PH * hpw));
        if constexpr (kLine) {
            // 64 lanes = TPI tokens x PPT pieces; wave w issues instructions 4w .. 4w + 3
            constexpr int PPT = 8 * HPW, TPI = 64 / PPT;
            const uint32_t l = lane_now();
    #pragma unroll
            for (int j = 4 * wave; j < 4 * wave + 4; ++j) {
                if (j * TPI >= valid) break;
                ++n;
                const int t = j * TPI + (int)(l / PPT);
                const int p = (int)(l % PPT) ^ swz(t);
                const uint32_t src = p < 4 * HPW ? (uint32_t)(SL.k_idx + 64 * h0 + 16 * p)
                                                 : (uint32_t)(SL.v_idx + 64 * h0 + 16 * (p - 4 * HPW));
                if (t < valid) copy16v(a.cache + d.off[t] + src, dst + j * 1024);
            }
        } else {
            for (int tt = wave; tt < valid; tt += hpw) {
                const uint8_t *tok = a.cache + readlane64(base, tt);  // uniform slot address
                if (lane < 2 * PH * hpw) copy16(tok, kv_src, dst + tt * TS);
                ++n;
            }
        }
        if constexpr (HPW >= 4) {
            // Norms in 16-byte pieces (4 heads' K or V norms of one token): piece p =
            // kind * NPH + sub (kind 0: K, 1: V; sub: heads 4 sub .. 4 sub + 3) of token t
            // lands at slot 32 p + t.  Copy c (wave c) moves pieces 2c and 2c + 1 of all
            // tokens: lane l takes token l & 31, piece 2c + (l >> 5).
            constexpr int NPH = HPW / 4;
            if (wave < NPH) {
                const uint32_t l = lane_now();  // lane-derived values rebuilt here, not kept live
                const int t = l & 31, p = 2 * wave + (int)(l >> 5);
                const int kind = p / NPH, sub = p % NPH;
                const uint32_t src = (kind ? (uint32_t)SL.v_norm : (uint32_t)SL.k_norm) + 4 * h0 + 16 * sub;
                if (t < valid) copy16v(a.cache + d.off[t] + src, dst + norm_off + 1024 * wave);
                ++n;
            }
        } else {
            // norm rows 2*wave, 2*wave+1 (row j < hpw: K norm of head h0+j, else V norm of head h0+j-hpw)
            const int nrow = 2 * wave + (lane >> 5);
            const uint32_t norm_src = nrow < hpw ? (uint32_t)(SL.k_norm + 4 * (h0 + nrow))
                                                 : (uint32_t)(SL.v_norm + 4 * (h0 + nrow - hpw));
            if (tl_copy < valid) copy4(a.cache + base + norm_src, dst + norm_off + 256 * wave);
            ++n;
        }
        return n;
    };
    // This wave's K (kind 0) or V (kind 1) norm of token t in stage sb.
    auto norm_at = [&](const uint8_t *sb, int kind, int t) {
        if constexpr (HPW >= 4) {
            constexpr int NPH = HPW / 4;
            return *reinterpret_cast<const float *>(sb + norm_off + 16 * ((kind * NPH + (wave >> 2)) * 32 + t) +
                                                    4 * (wave & 3));
        } else {
            return *reinterpret_cast<const float *>(sb + norm_off + 128 * (kind * hpw + wave) + 4 * t);
        }
    };

    // Query operand of sequence s -> the query slot (each wave its own kv head):
    // ceil(G / 4) 16-byte copies per wave.
    auto issue_q = [&](int s) {
        const uint8_t *src = reinterpret_cast<const uint8_t *>(a.qops) + ((int64_t)s * a.H + h0 + wave) * 16 * 256;
        const uint32_t dst = lds_addr(qarea + wave * G * 256);
        const uint32_t l16 = 16u * lane_now();
        for (int j = 0; j < G * 256; j += 1024)
            if (j + l16 < (uint32_t)(G * 256)) copy16(src, j + l16, dst + j);
        return (G + 3) / 4;
    };

    // The codebook loads are compiler-visible: issued before the descriptor copies
    // and covered by their wait, so no wait of the compiler's for them lands after
    // the first tile copies (it would wait for those too).
    float cbv = 0.f;
    if (threadIdx.x < 32) {
        const int e = threadIdx.x & 15;
        cbv = threadIdx.x < 16 ? (e < a.nkc ? a.kc[e] : 0.f) : (e < a.nvc ? a.vc[e] : 0.f);
    }
    for (int i = 0; i < min(nt, RING); ++i) issue_desc(i);
    wait_copies<0>();
    if (threadIdx.x < 32) cbarea[threadIdx.x] = cbv;
    __syncthreads();

    // Per-segment state.  No compiler-visible global load is issued inside the tile
    // loop: the compiler does not count the copies, so a wait it inserted for a load
    // of its own would wait for every copy in flight and stall the pipeline.  The
    // query operand therefore arrives by copy, in the same stream as the tiles.
    int seq = -1;
    u32x4 qop[4];
    constexpr int NACC = WIDE ? 8 : 4;
    f32x4 acc[NACC];  // [rb] (dims (first | second) of pair rb), WIDE: [rb] first dims, [4 + rb] second dims
    float m_run, l_run;
    int e_run;      // bf16: every V norm of the segment so far is < 2^e_run; acc carries 2^-e_run
    float lim;      // 2^e_run
    const float sc = a.score_scale;
    auto begin_segment = [&]() {
        const uint32_t ln = lane_now(), lc = ln & 15;  // rebuilt here, not kept live across the loop
        const uint32_t qc = WIDE ? lc : (lc & 7);      // query head of this lane's column
        const uint4 *src = reinterpret_cast<const uint4 *>(qarea + wave * G * 256 + qc * 256 + (ln >> 4) * 64);
    #pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 v = (int)qc < G ? src[c] : make_uint4(0, 0, 0, 0);
            qop[c] = u32x4{v.x, v.y, v.z, v.w};
        }
    #pragma unroll
        for (int m = 0; m < NACC; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
        m_run = -INFINITY;  // running max (log2 domain) for this lane's query head
        l_run = 0.f;        // this lane's partial sum of p
        // bf16: the V operand is V * 2^-e_run <= max|c| (fp16); starting at 2^-64 keeps
        // tiny norms representable until the first tile raises it.
        e_run = kScaleV ? -64 : 0;
        lim = kScaleV ? 0x1p-64f : INFINITY;
    };
    // Partial of the current segment -> slot w + seq: (m_run + e_run, l_run 2^-e_run, acc),
    // acc in head-dim order.  Addresses are a uniform 64-bit base plus a 32-bit lane
    // offset computed here (a hoisted 64-bit per-lane address would be spilled, and its
    // reload would wait for the copies in flight).
    auto end_segment = [&]() {
        const float lsum = rows_sum(l_run);
        const uint32_t ln = lane_now(), lc = ln & 15, lg = ln >> 4;
        const uint32_t qc = WIDE ? lc : (lc & 7);
        if ((int)qc < a.G) {
            const int64_t slot = (int64_t)(w + seq) * a.HQ + (h0 + wave) * a.G;  // uniform: query head h*G of the slot
            uint8_t *pa = reinterpret_cast<uint8_t *>(a.part_acc + slot * kD);
            uint8_t *pm = reinterpret_cast<uint8_t *>(a.part_ml + slot * 2);
            const uint32_t hoff = qc * kD * 4;
    #pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t r8 = 8 * (4 * lg + i);  // nibble dword 4g + i: dims 8r .. 8r+7
                if constexpr (WIDE) {
                    *reinterpret_cast<float4 *>(pa + hoff + 4 * r8) = make_float4(acc[0][i], acc[1][i], acc[4][i], acc[5][i]);
                    *reinterpret_cast<float4 *>(pa + hoff + 4 * (r8 + 4)) = make_float4(acc[2][i], acc[3][i], acc[6][i], acc[7][i]);
                } else {
                    const uint32_t d0 = r8 + (lc >= 8 ? 2 : 0);  // columns >= 8: the second dims of the pairs
                    *reinterpret_cast<float2 *>(pa + hoff + 4 * d0) = make_float2(acc[0][i], acc[1][i]);
                    *reinterpret_cast<float2 *>(pa + hoff + 4 * (d0 + 4)) = make_float2(acc[2][i], acc[3][i]);
                }
            }
            if (lg == 0 && (WIDE || lc < 8))
                *reinterpret_cast<float2 *>(pm + 8u * qc) = make_float2(m_run + (float)e_run, ldexpf(lsum, -e_run));
        }
    };
    // The query slot holds the operand of the segment starting at local tile q_upto;
    // the next one is copied once that segment has begun (its operand is then in
    // registers), before the tile copies of the same iteration, so the wait for the
    // tile that starts the new segment also covers it.
    int q_upto = 0;
    // Copy accounting (wave-uniform): cnt = copy instructions this wave issued since
    // the prologue's wait; tend[k] = cnt just after the copies of tile t + k (k < NS)
    // at the top of iteration t; qend = cnt just after the last query-operand copies.
    int cnt = issue_q(__builtin_amdgcn_readfirstlane(ring[0].seq));
    int qend = cnt;
    int tend[NS];
    #pragma unroll
    for (int k = 0; k < NS; ++k) {
        if (k < nt) cnt += issue(k, lds + k * stage_bytes);
        tend[k] = cnt;
    }
    // Most copies a wave can have in flight after the ones waited for: NS - 1 tiles,
    // their descriptors and one query operand.
    constexpr int kTileCopies = kLine ? 5 : (HPW > 0 ? (kTile + HPW - 1) / HPW + 1 : 12);
    constexpr int kMaxInFlight = (NS - 1) * (kTileCopies + 1) + 4 < 63 ? (NS - 1) * (kTileCopies + 1) + 4 : 63;

    int si = 0;  // stage of tile t (t % NS)
    for (int t = 0; t < nt; ++t) {
        uint8_t *const sb = lds + si * stage_bytes;
        // Tile t landed?  The copies issued after tile t's (those of tiles t+1 ..
        // t+NS-1, descriptors, a query operand) may stay in flight -- except the query
        // operand of a segment that starts at tile t.
        {
            // (the count is wave-uniform: read into a scalar register, the search over
            // the immediates is scalar compares and branches, not VALU compares and exec masks)
            const int need = q_upto == t ? max(tend[0], qend) : tend[0];
            wait_copies_upto<0, kMaxInFlight>(__builtin_amdgcn_readfirstlane(cnt - need));
        }
        __syncthreads();

        const int tseq = __builtin_amdgcn_readfirstlane(ring[t & (RING - 1)].seq);
        const int valid = __builtin_amdgcn_readfirstlane(ring[t & (RING - 1)].valid);
        if (tseq != seq) {  // a new sequence starts at this tile
            if (seq >= 0) end_segment();
            seq = tseq;
            begin_segment();
        }
        // ---- this wave's operands of the tile ------------------------------------
        // (lane-derived values of this section are rebuilt from the lane id here, so
        // that their addresses are not loop-invariant registers: under pressure those
        // are spilled, and a spill reload waits for every copy in flight)
        const uint32_t lnow = lane_now();
        const int col = (int)(lnow & 15), g = (int)(lnow >> 4), tl = (int)(lnow & 31), hh = (int)(lnow >> 5);
        // K: token col (and 16 + col), dims 32g .. 32g+31 (16 nibble bytes, or the
        // 12-byte dense group g)
        uint4 kw0, kw1;
        if constexpr (D3) {
            const uint8_t *kb = sb + col * TS + IB * wave + 12 * g;
            const uint32_t *k0p = reinterpret_cast<const uint32_t *>(kb);
            const uint32_t *k1p = reinterpret_cast<const uint32_t *>(kb + 16 * TS);
            kw0 = make_uint4(k0p[0], k0p[1], k0p[2], 0u);
            kw1 = make_uint4(k1p[0], k1p[1], k1p[2], 0u);
        } else {
            kw0 = *reinterpret_cast<const uint4 *>(sb + at(col, 4 * wave + g, 0));
            kw1 = *reinterpret_cast<const uint4 *>(sb + at(16 + col, 4 * wave + g, 0));
        }
        // V: nibble dword col (dims 8 col .. 8 col + 7) of the lane's 8 tokens 4g + i and
        // 16 + 4g + i, or dense: dword min(col % 4, 2) of group col / 4 (position 3 is
        // assembled from the quad's other lanes below)
        uint32_t vw[8];
        if constexpr (D3) {
            const uint8_t *vb = sb + 4 * g * TS + IB * hpw + IB * wave + 12 * (col >> 2) + 4 * min(col & 3, 2);
    #pragma unroll
            for (int i = 0; i < 8; ++i) vw[i] = *reinterpret_cast<const uint32_t *>(vb + (i < 4 ? i : 12 + i) * TS);
        } else {
    #pragma unroll
            for (int i = 0; i < 8; ++i)
                vw[i] = *reinterpret_cast<const uint32_t *>(
                    sb + at(i < 4 ? 4 * g + i : 12 + 4 * g + i, 4 * hpw + 4 * wave + (col >> 2), 4 * (col & 3)));
        }
        // the K and V norms of token tl (this lane's tables)
        float nk = norm_at(sb, 0, tl), nv = norm_at(sb, 1, tl);

        // ---- tokens past the end were not copied: their stage bytes are stale.  Zero
        // their norms (their tables are then zero) and V index dwords (a stale nibble
        // >= 8 would look up a non-zero byte pattern, and NaN * 0 would reach the
        // accumulator); their scores are masked below.
        if (valid < kTile) {
            // (each masking block takes `valid` through an empty asm, so that its
            // compares stay inside the block instead of running for every full tile)
            const int vv = opaque_s(valid);
            const uint32_t ln = lane_now();
            const int g4 = 4 * (int)(ln >> 4);  // 4g, rebuilt here (not kept live)
            const int t32 = (int)(ln & 31);
            nk = t32 < vv ? nk : 0.f;
            nv = t32 < vv ? nv : 0.f;
    #pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int tt = i < 4 ? g4 + i : 12 + g4 + i;
                vw[i] = tt < vv ? vw[i] : 0u;
            }
        }
        // bf16: a V norm at or above 2^e_run (rare after the first tile): raise e_run to
        // the tile's largest norm and rescale acc, which carries 2^-e_run.
        if constexpr (kScaleV) {
            if (__any(nv >= lim)) {
                float nvm = rows_max(nv);
    #pragma unroll
                for (int o = 1; o < 16; o <<= 1) nvm = fmaxf(nvm, __shfl_xor(nvm, o));
                const int e_tile = (int)((__float_as_uint(nvm) >> 23) & 0xffu) - 126;  // 2^e_tile > max norm
                if (e_tile > e_run) {
                    const float f = ldexpf(1.f, e_run - e_tile);
    #pragma unroll
                    for (int m = 0; m < NACC; ++m) acc[m] *= f;
                    e_run = e_tile;
                    lim = ldexpf(1.f, e_run);
                }
            }
        }
        // ---- codebook tables of token tl: this lane's half of the K table (q dtype) and
        // of the V table (fp16 image), written over the wave's own K index bytes of the
        // token, which were read above (LDS instructions of a wave complete in order)
        // Tables of token t: K in K index pieces 0 (and 1) of the wave's head, V in pieces
        // 2 (and 3); dense layout: K at byte 0, V at byte 16 of the head's 48 bytes.
        auto tab_k = [&](int t, int q) { return sb + (D3 ? t * TS + IB * wave + 16 * q : at(t, 4 * wave + q, 0)); };
        auto tab_v = [&](int t, int q) { return sb + (D3 ? t * TS + IB * wave + 16 + 16 * q : at(t, 4 * wave + 2 + q, 0)); };
        table_half<DT, KB, false>(cbarea, nk, hh, tab_k(tl, 0), tab_k(tl, 1));
        table_half<DT, VB, true>(cbarea + 16, kScaleV ? ldexpf(nv, -e_run) : nv, hh, tab_v(tl, 0), tab_v(tl, 1));
        __builtin_amdgcn_wave_barrier();
        const Table16 tk0 = read_table<KB>(tab_k(col, 0), tab_k(col, 1));
        const Table16 tk1 = read_table<KB>(tab_k(16 + col, 0), tab_k(16 + col, 1));
        // ---- V operands: token i's dims of the lane's nibble dword, by pair:
        //   av[i] = (e0 e2) (e1 e3) (e4 e6) (e5 e7)
        // Index selectors (one index per byte) of the even and the odd dims.  Dense:
        // lanes of positions 0..2 mask their own bytes; the position-3 lane takes the
        // top bits of its quad's A, B and C lanes (same token): one form for all lanes,
        // (x >> s1) & m1 | (y >> s2) & m2, with per-lane shifts and masks.
        auto sel = [&](uint32_t x, uint32_t &ev, uint32_t &od) {
            if constexpr (D3) {
                const bool p3 = (col & 3) == 3;
                const uint32_t xe = quad_pick<0x24>(x), xo = quad_pick<0x64>(x), y = quad_pick<0xa4>(x);
                const uint32_t m1 = p3 ? 0x03030303u : 0x07070707u, m2 = p3 ? 0x04040404u : 0u;
                ev = ((xe >> (p3 ? 6 : 0)) & m1) | ((y >> 4) & m2);
                od = ((xo >> (p3 ? 6 : 3)) & m1) | ((y >> 5) & m2);
            } else {
                ev = (x >> 4) & 0x0f0f0f0fu;
                od = x & 0x0f0f0f0fu;
            }
        };
        u32x4 av[8];
    #pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int ti = i < 4 ? 4 * g + i : 12 + 4 * g + i;
            const Table16 tv = read_table<VB>(tab_v(ti, 0), tab_v(ti, 1));
            uint32_t ev, od;
            sel(vw[i], ev, od);
            const uint2 e = lookup4<VB>(tv, ev), o = lookup4<VB>(tv, od);
            av[i] = u32x4{e.x, o.x, e.y, o.y};
        }
        __syncthreads();  // the stage and descriptor slot t are free once every wave holds its operands

        // ---- next query operand, descriptor t+RING and tile t+NS ---------------------
        if (q_upto <= t && t + 1 < nt) {
            const int s1 = __builtin_amdgcn_readfirstlane(ring[(t + 1) & (RING - 1)].seq);
            if (s1 != seq) {
                cnt += issue_q(s1);
                qend = cnt;
                q_upto = t + 1;
            } else if (t + 2 < nt) {
                const int s2 = __builtin_amdgcn_readfirstlane(ring[(t + 2) & (RING - 1)].seq);
                if (s2 != s1) {
                    cnt += issue_q(s2);
                    qend = cnt;
                    q_upto = t + 2;
                }
            }
        }
        if (t + RING < nt) cnt += issue_desc(t + RING);
        if (t + NS < nt) cnt += issue(t + NS, sb);
    #pragma unroll
        for (int k = 0; k + 1 < NS; ++k) tend[k] = tend[k + 1];
        tend[NS - 1] = cnt;
        si = si + 1 == NS ? 0 : si + 1;

        // ---- S^T = K Q^T (exact products of the q-dtype values, fp32 sums) -----------
        f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = s0;
        if constexpr (D3) {
            // dense group (A, B, C): positions 0..2 from their own dword, 3 from the top bits
            const uint32_t a0[3] = {kw0.x, kw0.y, kw0.z}, a1[3] = {kw1.x, kw1.y, kw1.z};
    #pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t e0 = c < 3 ? d3_even(a0[c]) : d3_even3(a0[0], a0[2]);
                const uint32_t o0 = c < 3 ? d3_odd(a0[c]) : d3_odd3(a0[1], a0[2]);
                const uint32_t e1 = c < 3 ? d3_even(a1[c]) : d3_even3(a1[0], a1[2]);
                const uint32_t o1 = c < 3 ? d3_odd(a1[c]) : d3_odd3(a1[1], a1[2]);
                s0 = mfma<DT>(decode_row8_sel<KB>(tk0, e0, o0), qop[c], s0);
                s1 = mfma<DT>(decode_row8_sel<KB>(tk1, e1, o1), qop[c], s1);
            }
        } else {
            const uint32_t k0w[4] = {kw0.x, kw0.y, kw0.z, kw0.w};
            const uint32_t k1w[4] = {kw1.x, kw1.y, kw1.z, kw1.w};
    #pragma unroll
            for (int c = 0; c < 4; ++c) {
                s0 = mfma<DT>(decode_row8<KB>(tk0, k0w[c]), qop[c], s0);
                s1 = mfma<DT>(decode_row8<KB>(tk1, k1w[c]), qop[c], s1);
            }
        }
        // ---- mask, online softmax ------------------------------------------------------
        // The score scale sc > 0 enters the exponent's fma (and the max, which it
        // commutes with).
        float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        if (valid < kTile) {
            const int vv = opaque_s(valid);
            const int g4 = 4 * (int)(lane_now() >> 4);
    #pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int tt = i < 4 ? g4 + i : 12 + g4 + i;
                s[i] = tt < vv ? s[i] : -INFINITY;
            }
        }
        float tmax = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
        tmax = rows_max(tmax) * sc;
        // Lazy running max: rescale only when a column's max exceeds m_run by more
        // than 8 (log2 units).  In between, p = 2^(score - m_run) <= 2^8, so the fp16
        // P operand stays in range; acc and l_run are relative to the same m_run, so
        // the result does not depend on when the rescale happens.
        if (__any(tmax > m_run + 8.f)) {
            const float m_new = fmaxf(m_run, tmax);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // m_run = -inf on the first tile -> 0
    #pragma unroll
            for (int m = 0; m < NACC; ++m) acc[m] *= alpha;
            l_run *= alpha;
            m_run = m_new;
        }
        float p[8];
    #pragma unroll
        for (int i = 0; i < 8; ++i) {
            p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], sc, -m_run));
            l_run += p[i];
        }

        // ---- O^T += V^T P^T ---------------------------------------------------
        // P^T k slots 8g + 2i, +1 (token 16kb + 4g + i; the two dims of a pair):
        // (p, 0) in columns < 8 and (0, p) in columns >= 8, or (WIDE) both.
        const uint32_t x01 = pack2<RQ_DTYPE_F16>(p[0], p[1]), x23 = pack2<RQ_DTYPE_F16>(p[2], p[3]);
        const uint32_t x45 = pack2<RQ_DTYPE_F16>(p[4], p[5]), x67 = pack2<RQ_DTYPE_F16>(p[6], p[7]);
        if constexpr (!WIDE) {
            const bool hi_col = (lane_now() & 8) != 0;
            const uint32_t se = hi_col ? 0x01000c0cu : 0x0c0c0100u;  // element 0 -> (x, 0) or (0, x)
            const uint32_t so = hi_col ? 0x03020c0cu : 0x0c0c0302u;  // element 1
            const u32x4 b0 = u32x4{perm(x01, x01, se), perm(x01, x01, so), perm(x23, x23, se), perm(x23, x23, so)};
            const u32x4 b1 = u32x4{perm(x45, x45, se), perm(x45, x45, so), perm(x67, x67, se), perm(x67, x67, so)};
    #pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                acc[rb] = mfma<RQ_DTYPE_F16>(u32x4{av[0][rb], av[1][rb], av[2][rb], av[3][rb]}, b0, acc[rb]);
                acc[rb] = mfma<RQ_DTYPE_F16>(u32x4{av[4][rb], av[5][rb], av[6][rb], av[7][rb]}, b1, acc[rb]);
            }
        } else {
            const u32x4 b0e = u32x4{x01 & 0xffffu, x01 >> 16, x23 & 0xffffu, x23 >> 16};
            const u32x4 b1e = u32x4{x45 & 0xffffu, x45 >> 16, x67 & 0xffffu, x67 >> 16};
            const u32x4 b0o = u32x4{x01 << 16, x01 & 0xffff0000u, x23 << 16, x23 & 0xffff0000u};
            const u32x4 b1o = u32x4{x45 << 16, x45 & 0xffff0000u, x67 << 16, x67 & 0xffff0000u};
    #pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const u32x4 a0 = u32x4{av[0][rb], av[1][rb], av[2][rb], av[3][rb]};
                const u32x4 a1 = u32x4{av[4][rb], av[5][rb], av[6][rb], av[7][rb]};
                acc[rb] = mfma<RQ_DTYPE_F16>(a0, b0e, acc[rb]);
                acc[rb] = mfma<RQ_DTYPE_F16>(a1, b1e, acc[rb]);
                acc[4 + rb] = mfma<RQ_DTYPE_F16>(a0, b0o, acc[4 + rb]);
                acc[4 + rb] = mfma<RQ_DTYPE_F16>(a1, b1o, acc[4 + rb]);
            }
        }
    }

    end_segment();
}

// Segments per merge pass (PASS = 16 or 32): lane c < PASS loads segment c's (m, l),
// and every lane loads its two dims of all of them before any is used (one load
// round per pass).  32 halves the rounds of long sequences; 16 needs ~65 fewer
// VGPRs, so more merge waves are resident at once.

// Merge the partials of (seq, query head): log-sum-exp over the segments, round
// to the query dtype (the reference's out_rot, fused_paged_rq_decode.py:201-206),
// rotate back by R in fp32 and round again (:308).  One wave per query head,
// two head dims per lane; per pass of kMergePass segments, the (m, l) of each segment
// and the lane's accumulator entries of all of them are loaded together.
// kSplit == 1: a workgroup holds up to four query heads, one wave each.  kSplit > 1
// (few (sequence, head) pairs, each with many segments): the kSplit waves of a
// workgroup share one query head, wave i taking segment passes i, i + kSplit, ...,
// and wave 0 combines their (max, sum, accumulator) states through LDS -- one
// round of loads instead of a chain of passes, on kSplit times as many waves.
template <int DT, int kMergePass, int kSplit>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    static_assert(kSplit == 1 || kSplit == 4, "one wave per head, or four (the 256-thread block)");
    const int64_t seq = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int hq = kSplit == 1 ? blockIdx.x * (blockDim.x >> 6) + wave : blockIdx.x;
    const int share = kSplit == 1 ? 0 : wave;  // first segment pass of this wave
    __shared__ float orot_all[4][kD];
    float *orot = orot_all[wave];
    if (hq >= a.HQ) return;  // (kSplit > 1: the whole workgroup or none of it)
    // R entries for this lane's two output dims (issued first; independent of the partials)
    float rr[2][4];
    #pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int d = 2 * lane + e;
        const int k0 = (d / a.rot_block) * a.rot_block;
    #pragma unroll
        for (int i = 0; i < 4; ++i) rr[e][i] = i < a.rot_block && share == 0 ? a.R[(k0 + i) * kD + d] : 0.f;
    }
    // Workgroups whose tile ranges cover the sequence (found by the prep kernel):
    // partials sit at slots w + seq for w in [w_lo, w_lo + nch); workgroups with an
    // empty range (more workgroups than tiles) wrote nothing.
    // (the prep kernel does not run when no sequence has tokens: then nch = 0)
    // The merge is a short chain of dependent loads, so the words it needs first are
    // loaded together, unconditionally (they are in-bounds workspace words, written by
    // the prep kernel for every sequence), and used only when the sequence has tiles.
    const int tp_lo = a.tile_prefix[2 * seq], tp_n = a.tile_prefix[2 * seq + 1];
    const int ntt = *a.n_tiles_total;
    const int n = seq_tiles(a, seq);
    const int w_lo = n > 0 ? tp_lo : 0, nch = n > 0 ? tp_n : 0;
    const RangeSplit rsp = make_split(a, ntt);
    auto has_tiles = [rsp](int w) { return range_start(rsp, w + 1) > range_start(rsp, w); };
    const float *ml = a.part_ml + (w_lo + seq) * (int64_t)a.HQ * 2 + hq * 2;
    const float *pa = a.part_acc + (w_lo + seq) * (int64_t)a.HQ * kD + hq * kD;
    const int64_t cs_ml = (int64_t)a.HQ * 2, cs_acc = (int64_t)a.HQ * kD;
    float lsum = 0.f, o0 = 0.f, o1 = 0.f, M = -INFINITY;
    for (int c0 = share * kMergePass; c0 < nch; c0 += kSplit * kMergePass) {
        // lane c (< kMergePass) loads segment c0 + c's (m, l); every lane loads its two
        // dims of up to kMergePass segments' accumulators -- all issued before any is used
        const int c = c0 + (lane & (kMergePass - 1));
        const bool ok = c < nch && has_tiles(w_lo + c);
        const uint64_t okm = __ballot(ok && lane < kMergePass);
        const float2 v = ok ? *reinterpret_cast<const float2 *>(ml + c * cs_ml) : make_float2(-INFINITY, 0.f);
        float2 x[kMergePass];
    #pragma unroll
        for (int u = 0; u < kMergePass; ++u)
            x[u] = (okm >> u) & 1 ? reinterpret_cast<const float2 *>(pa + (c0 + u) * cs_acc)[lane] : make_float2(0.f, 0.f);
        float pm = lane < kMergePass ? v.x : -INFINITY;
        for (int o = kMergePass / 2; o >= 1; o >>= 1) pm = fmaxf(pm, __shfl_xor(pm, o));
        pm = __shfl(pm, 0);
        const float Mn = fmaxf(M, pm);
        // -inf - finite -> 0 on the first pass; 1 while every segment seen has an empty
        // range (M = Mn = -inf: a wave whose passes begin among such segments)
        const float alpha = M == Mn ? 1.f : __builtin_amdgcn_exp2f(M - Mn);
        o0 *= alpha;
        o1 *= alpha;
        lsum *= alpha;
        M = Mn;
        const float w = ok && lane < kMergePass ? __builtin_amdgcn_exp2f(v.x - M) : 0.f;
        float wl = w * v.y;
        for (int o = kMergePass / 2; o >= 1; o >>= 1) wl += __shfl_xor(wl, o);
        lsum += __shfl(wl, 0);
    #pragma unroll
        for (int u = 0; u < kMergePass; ++u) {
            const float wu = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), u));
            o0 += wu * x[u].x;
            o1 += wu * x[u].y;
        }
    }
    if constexpr (kSplit > 1) {
        // each wave's state relative to its own max M_i (-inf, sum 0, accumulator 0 for a
        // wave without segments); wave 0 rescales them to the overall max and adds them up
        __shared__ float2 st_acc[kSplit][kD / 2];
        __shared__ float2 st_ml[kSplit];
        st_acc[wave][lane] = make_float2(o0, o1);
        if (lane == 0) st_ml[wave] = make_float2(M, lsum);
        __syncthreads();
        if (wave != 0) return;
        float2 ml[kSplit];
        float Mt = -INFINITY;
    #pragma unroll
        for (int i = 0; i < kSplit; ++i) {
            ml[i] = st_ml[i];
            Mt = fmaxf(Mt, ml[i].x);
        }
        lsum = o0 = o1 = 0.f;
    #pragma unroll
        for (int i = 0; i < kSplit; ++i) {
            const float f = ml[i].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml[i].x - Mt);
            const float2 x = st_acc[i][lane];
            lsum += f * ml[i].y;
            o0 += f * x.x;
            o1 += f * x.y;
        }
    }
    const float inv = nch > 0 ? 1.f / lsum : 0.f;  // empty context -> zeros (reference: acc 0, l 1)
    orot[2 * lane] = Elem<DT>::to_f32(Elem<DT>::from_f32(o0 * inv));
    orot[2 * lane + 1] = Elem<DT>::to_f32(Elem<DT>::from_f32(o1 * inv));
    __builtin_amdgcn_wave_barrier();
    uint16_t *dst = reinterpret_cast<uint16_t *>(a.out) + seq * a.o_ss + (int64_t)hq * a.o_sh;
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int d = 2 * lane + e;
        const int k0 = (d / a.rot_block) * a.rot_block;
        float r = 0.f;
        for (int i = 0; i < a.rot_block; ++i) r = __builtin_fmaf(orot[k0 + i], rr[e][i], r);
        packed |= Elem<DT>::from_f32(r) << (16 * e);
    }
    reinterpret_cast<uint32_t *>(dst)[lane] = packed;
}

// Bound on decode workgroups per CU.  One-wave workgroups (one kv head: a
// tensor-parallel slice) take up to 8 per CU (TP-8 slice of config 1: 32.9 us
// against 34.1 at 4 and 36.8 at 16, where the first copies of all workgroups become
// one burst); both index layouts fit 8 of them in LDS, so they get the same grid and
// the same result bit for bit.  Wider ones take at most 4 (two per CU at 8 kv heads,
// by LDS).  The partial slots of the workspace are sized by the query heads alone
// (the workspace query does not know the kv heads): 8 per CU when num_q_heads <= 16,
// which covers every one-head launch (its query heads are its GQA group, <= 16);
// otherwise 4.
constexpr int decode_wg_cap(int hpw, int64_t num_q_heads) { return hpw == 1 && num_q_heads <= 16 ? 8 : 4; }
constexpr int decode_slot_factor(int64_t num_q_heads) { return num_q_heads <= 16 ? 8 : 4; }

// Resident decode workgroups per CU for an LDS size (cached per device and size;
// the cache of each kernel instance is guarded by a mutex, so concurrent callers
// see whole entries).
template <int DT, int KB, int VB, int HPW, bool D3, bool WIDE>
static int decode_per_cu(const DecodeArgs &a, size_t lds) {
    static int cache[64][8][2] = {};  // [device][entry] = {lds, workgroups per CU}
    static std::mutex mu;
    int dev = 0;
    (void)hipGetDevice(&dev);
    dev = dev < 0 || dev >= 64 ? 0 : dev;
    {
        std::lock_guard<std::mutex> lock(mu);
        for (auto &e : cache[dev])
            if (e[0] == (int)lds && e[1] > 0) return e[1];
    }
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &nb, reinterpret_cast<const void *>(&decode_kernel<DT, KB, VB, HPW, D3, WIDE>), 64 * a.hpw, lds) !=
            hipSuccess ||
        nb <= 0)
        nb = 1;
    nb = std::min(nb, decode_wg_cap(a.hpw, a.HQ));
    std::lock_guard<std::mutex> lock(mu);
    for (auto &e : cache[dev]) {
        if (e[0] == (int)lds && e[1] > 0) break;  // another caller stored it meanwhile
        if (e[1] == 0) {
            e[0] = (int)lds;
            e[1] = nb;
            break;
        }
    }
    return nb;
}

// Events recorded at the decode kernel's own start and end (rq_fused_decode_timed), or none.
struct KernelEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};

// configure: set the grid and range split only (before the prep kernel, which
// needs them); otherwise launch.
template <int DT, int KB, int VB, int HPW, bool D3, bool WIDE>
static void launch_decode_h(DecodeArgs &a, size_t lds, hipStream_t st, bool configure, KernelEvents ev) {
    if (!configure) {
        const dim3 grid((unsigned)a.grid_w, 1, a.H / a.hpw), block(64 * a.hpw);
        if (ev.start != nullptr || ev.stop != nullptr)  // events at this kernel's own start and end
            hipExtLaunchKernelGGL((decode_kernel<DT, KB, VB, HPW, D3, WIDE>), grid, block, lds, st, ev.start, ev.stop, 0,
                                  a);
        else
            hipLaunchKernelGGL((decode_kernel<DT, KB, VB, HPW, D3, WIDE>), grid, block, lds, st, a);
        return;
    }
    // as many workgroups per kv-head group as are resident at once
    const int per_cu = decode_per_cu<DT, KB, VB, HPW, D3, WIDE>(a, lds);
    const int groups = a.H / a.hpw;
    a.grid_w = std::max(1, per_cu * device_cus() / groups);
    // rank weights by workgroups per CU (workgroups [r CUs, (r+1) CUs) are
    // dispatched r-th onto each CU)
    // (two per CU: 65:35, the best of a sweep on config 1; three: 44:28:28, on config 4's
    // decodes 202.8-206.8 us against 213.4-215.1 at equal weights, 40:30:30 206.9-210.5,
    // 50:25:25 214.9-216.1)
    static const int kRankWt[5][4] = {{1, 1, 1, 1}, {1, 1, 1, 1}, {65, 35, 35, 35}, {44, 28, 28, 28}, {1, 1, 1, 1}};
    const int pc = groups == 1 ? std::min(per_cu, 4) : 1;
    a.split_c = pc > 1 ? a.grid_w / pc : a.grid_w;
    uint64_t tot = 0;
    for (int r = 0; r < 4; ++r) {
        a.wt[r] = kRankWt[pc][r];
        const int n_r = r < 3 ? std::max(0, std::min(a.split_c, a.grid_w - r * a.split_c)) : std::max(0, a.grid_w - 3 * a.split_c);
        tot += (uint64_t)n_r * a.wt[r];
    }
    a.split_r = UINT64_MAX / tot;
}

template <int DT, int KB, int VB, bool D3, bool WIDE>
static void launch_decode_w(DecodeArgs &a, size_t lds, hipStream_t st, bool configure, KernelEvents ev) {
    if (a.hpw == 8) launch_decode_h<DT, KB, VB, 8, D3, WIDE>(a, lds, st, configure, ev);
    else if (a.hpw == 4) launch_decode_h<DT, KB, VB, 4, D3, WIDE>(a, lds, st, configure, ev);
    else if (a.hpw == 2) launch_decode_h<DT, KB, VB, 2, D3, WIDE>(a, lds, st, configure, ev);
    else if (a.hpw == 1) launch_decode_h<DT, KB, VB, 1, D3, WIDE>(a, lds, st, configure, ev);
    else launch_decode_h<DT, KB, VB, 0, D3, WIDE>(a, lds, st, configure, ev);
}

template <int DT, int KB, int VB, bool D3 = false>
static void launch_decode(DecodeArgs &a, size_t lds, hipStream_t st, bool configure, KernelEvents ev) {
    if (a.G > 8) launch_decode_w<DT, KB, VB, D3, true>(a, lds, st, configure, ev);
    else launch_decode_w<DT, KB, VB, D3, false>(a, lds, st, configure, ev);
}

template <int DT>
static void launch_decode_bits(DecodeArgs &a, size_t lds, int kb, int vb, bool dense3, hipStream_t st,
                               bool configure, KernelEvents ev) {
    if (dense3) launch_decode<DT, 3, 3, true>(a, lds, st, configure, ev);  // the layout holds 3-bit indices only
    else if (kb == 3 && vb == 3) launch_decode<DT, 3, 3>(a, lds, st, configure, ev);
    else if (kb == 3) launch_decode<DT, 3, 4>(a, lds, st, configure, ev);
    else if (vb == 3) launch_decode<DT, 4, 3>(a, lds, st, configure, ev);
    else launch_decode<DT, 4, 4>(a, lds, st, configure, ev);
}

// Workspace layout (256-byte aligned regions).
struct DecodeWorkspace {
    int64_t part_acc, part_ml, qops, descs, tile_prefix, n_tiles, total;
    DecodeWorkspace(int64_t num_seqs, int64_t num_q_heads, int64_t max_seq_len) {
        auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
        const int64_t slots = (int64_t)decode_slot_factor(num_q_heads) * device_cus() + num_seqs;
        const int64_t max_tiles = num_seqs * ((max_seq_len + kTile - 1) / kTile);
        part_acc = 0;
        part_ml = al(part_acc + slots * num_q_heads * kD * 4);
        qops = al(part_ml + slots * num_q_heads * 2 * 4);
        descs = al(qops + num_seqs * num_q_heads * 64 * 16 * 4);  // kv heads <= query heads
        tile_prefix = al(descs + max_tiles * (int64_t)sizeof(TileDesc));
        n_tiles = al(tile_prefix + num_seqs * 8);  // NT (int) at +0, range-split multiplier (uint64) at +8
        total = al(n_tiles + 16);
    }
};

}  // namespace rq

using namespace rq;

extern "C" int64_t rq_fused_decode_workspace_bytes(int64_t num_seqs, int32_t num_q_heads, int32_t head_dim,
                                                   int64_t max_seq_len) {
    (void)head_dim;
    return DecodeWorkspace(num_seqs, num_q_heads, std::max<int64_t>(max_seq_len, 1)).total;
}

static int fused_decode_impl(const void *q, int32_t dtype, int64_t num_seqs, int32_t num_q_heads,
                             int64_t q_stride_seq, int64_t q_stride_head, const uint8_t *kv_cache,
                             int64_t num_blocks, int32_t block_size, int64_t stride_block, int64_t stride_token,
                             int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                             const int32_t *block_table, int64_t max_blocks,
                             int64_t bt_stride_seq, const int32_t *seq_lens, int64_t max_seq_len,
                             const float *k_centroids, int32_t n_k_centroids, const float *v_centroids,
                             int32_t n_v_centroids, const float *rotation, int32_t rot_block, float sm_scale,
                             void *out, int64_t out_stride_seq, int64_t out_stride_head, void *workspace,
                             int64_t workspace_bytes, void *stream, KernelEvents ev = {});

extern "C" int rq_fused_decode(const void *q, int32_t dtype, int64_t num_seqs, int32_t num_q_heads,
                               int64_t q_stride_seq, int64_t q_stride_head, const uint8_t *kv_cache,
                               int64_t num_blocks, int32_t block_size, int64_t stride_block, int64_t stride_token,
                               int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                             const int32_t *block_table, int64_t max_blocks,
                               int64_t bt_stride_seq, const int32_t *seq_lens, int64_t max_seq_len,
                               const float *k_centroids, int32_t n_k_centroids, const float *v_centroids,
                               int32_t n_v_centroids, const float *rotation, int32_t rot_block, float sm_scale,
                               void *out, int64_t out_stride_seq, int64_t out_stride_head, void *workspace,
                               int64_t workspace_bytes, void *stream) {
    return fused_decode_impl(q, dtype, num_seqs, num_q_heads, q_stride_seq, q_stride_head, kv_cache, num_blocks,
                             block_size, stride_block, stride_token, num_kv_heads, head_dim, index_layout, block_table,
                             max_blocks,
                             bt_stride_seq, seq_lens, max_seq_len, k_centroids, n_k_centroids, v_centroids,
                             n_v_centroids, rotation, rot_block, sm_scale, out, out_stride_seq, out_stride_head,
                             workspace, workspace_bytes, stream);
}

extern "C" int rq_fused_decode_timed(const void *q, int32_t dtype, int64_t num_seqs, int32_t num_q_heads,
                                     int64_t q_stride_seq, int64_t q_stride_head, const uint8_t *kv_cache,
                                     int64_t num_blocks, int32_t block_size, int64_t stride_block,
                                     int64_t stride_token, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t index_layout, const int32_t *block_table, int64_t max_blocks,
                                     int64_t bt_stride_seq, const int32_t *seq_lens, int64_t max_seq_len,
                                     const float *k_centroids, int32_t n_k_centroids, const float *v_centroids,
                                     int32_t n_v_centroids, const float *rotation, int32_t rot_block, float sm_scale,
                                     void *out, int64_t out_stride_seq, int64_t out_stride_head, void *workspace,
                                     int64_t workspace_bytes, void *stream, void *event_start, void *event_stop) {
    KernelEvents ev;
    ev.start = (hipEvent_t)event_start;
    ev.stop = (hipEvent_t)event_stop;
    return fused_decode_impl(q, dtype, num_seqs, num_q_heads, q_stride_seq, q_stride_head, kv_cache, num_blocks,
                             block_size, stride_block, stride_token, num_kv_heads, head_dim, index_layout, block_table,
                             max_blocks, bt_stride_seq, seq_lens, max_seq_len, k_centroids, n_k_centroids,
                             v_centroids, n_v_centroids, rotation, rot_block, sm_scale, out, out_stride_seq,
                             out_stride_head, workspace, workspace_bytes, stream, ev);
}

// ---------------------------------------------------------------------------
// Allocation-free variant: the workspace is a file-scope device array.
// ---------------------------------------------------------------------------

namespace rq {
// Each GPU the library runs on holds its own copy of this array (its code
// object's global segment) until the process ends.  Host code never passes the
// array's name to a kernel or a copy: in host code the name is only a stand-in,
// and its device address, found once per device by hipGetSymbolAddress, is the
// one kept in g_scratch_ptr and used.
static __device__ __align__(256) uint8_t scratch[RQ_DECODE_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
static void *g_scratch_ptr[kMaxDevices] = {};
static std::mutex g_scratch_mutex;

// Device address of this device's scratch array (looked up on the first call on
// each device, with that device current).  nullptr with the error text set on failure.
static void *device_scratch() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("rq_fused_decode_noalloc: no current HIP device (or device id >= %d)", kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr) {
            set_error("rq_fused_decode_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                      hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}
}  // namespace rq

extern "C" int rq_fused_decode_noalloc(const void *q, int32_t dtype, int64_t num_seqs, int32_t num_q_heads,
                                       int64_t q_stride_seq, int64_t q_stride_head, const uint8_t *kv_cache,
                                       int64_t num_blocks, int32_t block_size, int64_t stride_block,
                                       int64_t stride_token, int32_t num_kv_heads, int32_t head_dim,
                                       int32_t index_layout, const int32_t *block_table, int64_t max_blocks,
                                       int64_t bt_stride_seq,
                                       const int32_t *seq_lens, int64_t max_seq_len, const float *k_centroids,
                                       int32_t n_k_centroids, const float *v_centroids, int32_t n_v_centroids,
                                       const float *rotation, int32_t rot_block, float sm_scale, void *out,
                                       int64_t out_stride_seq, int64_t out_stride_head, void *stream) {
    const int64_t need = rq_fused_decode_workspace_bytes(num_seqs, num_q_heads, head_dim, max_seq_len);
    if (need > RQ_DECODE_SCRATCH_BYTES) {
        set_error("rq_fused_decode_noalloc: %lld sequences x %d query heads up to %lld tokens need %lld bytes of "
                  "scratch, more than the library's static %lld (use rq_fused_decode with a workspace)",
                  (long long)num_seqs, num_q_heads, (long long)max_seq_len, (long long)need,
                  (long long)RQ_DECODE_SCRATCH_BYTES);
        return RQ_ENOSPACE;
    }
    void *ws = device_scratch();
    if (ws == nullptr) return RQ_ELAUNCH;
    return fused_decode_impl(q, dtype, num_seqs, num_q_heads, q_stride_seq, q_stride_head, kv_cache, num_blocks,
                             block_size, stride_block, stride_token, num_kv_heads, head_dim, index_layout, block_table,
                             max_blocks,
                             bt_stride_seq, seq_lens, max_seq_len, k_centroids, n_k_centroids, v_centroids,
                             n_v_centroids, rotation, rot_block, sm_scale, out, out_stride_seq, out_stride_head, ws,
                             RQ_DECODE_SCRATCH_BYTES, stream);
}

// Shared body of the two entry points (workspace given or the static scratch).
static int fused_decode_impl(const void *q, int32_t dtype, int64_t num_seqs, int32_t num_q_heads,
                             int64_t q_stride_seq, int64_t q_stride_head, const uint8_t *kv_cache,
                             int64_t num_blocks, int32_t block_size, int64_t stride_block, int64_t stride_token,
                             int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                             const int32_t *block_table, int64_t max_blocks,
                             int64_t bt_stride_seq, const int32_t *seq_lens, int64_t max_seq_len,
                             const float *k_centroids, int32_t n_k_centroids, const float *v_centroids,
                             int32_t n_v_centroids, const float *rotation, int32_t rot_block, float sm_scale,
                             void *out, int64_t out_stride_seq, int64_t out_stride_head, void *workspace,
                             int64_t workspace_bytes, void *stream, KernelEvents ev) {
    RQ_CHECK_ARG(dtype == RQ_DTYPE_BF16 || dtype == RQ_DTYPE_F16, "decode dtype must be f16 or bf16");
    RQ_CHECK_ARG(head_dim == kD, "head_dim %d unsupported (only %d)", head_dim, kD);
    RQ_CHECK_ARG(num_kv_heads >= 1 && num_kv_heads <= kMaxKvHeads, "num_kv_heads %d must be 1..%d", num_kv_heads,
                 kMaxKvHeads);
    RQ_CHECK_ARG(num_q_heads % num_kv_heads == 0 && num_q_heads / num_kv_heads <= 16,
                 "num_q_heads %d / num_kv_heads %d must be an integer <= 16", num_q_heads, num_kv_heads);
    RQ_CHECK_ARG((n_k_centroids == 8 || n_k_centroids == 16) && (n_v_centroids == 8 || n_v_centroids == 16),
                 "centroid counts must be 8 or 16");
    RQ_CHECK_ARG(rot_block == 2 || rot_block == 4, "rot_block %d must be 2 or 4", rot_block);
    RQ_CHECK_ARG(num_seqs >= 0 && max_seq_len >= 0 && block_size >= 1 && max_blocks >= 0, "bad sizes");
    const int lrc = check_index_layout(index_layout, head_dim, n_k_centroids, n_v_centroids);
    if (lrc) return lrc;
    const bool dense3 = index_layout == RQ_INDEX_DENSE3;
    RQ_CHECK_ARG(max_seq_len <= max_blocks * block_size, "max_seq_len exceeds block table capacity");
    RQ_CHECK_ARG(stride_token % 16 == 0 && stride_block % 16 == 0 && ((uintptr_t)kv_cache % 16) == 0,
                 "cache slots must be 16-byte aligned");
    RQ_CHECK_ARG(((uintptr_t)q % 16) == 0 && (q_stride_head * 2) % 16 == 0 && (q_stride_seq * 2) % 16 == 0,
                 "q rows must be 16-byte aligned");
    RQ_CHECK_ARG(((uintptr_t)k_centroids % 16) == 0 && ((uintptr_t)v_centroids % 16) == 0 && ((uintptr_t)rotation % 16) == 0,
                 "centroids and rotation must be 16-byte aligned");
    if (num_seqs == 0) return RQ_OK;
    RQ_CHECK_SPACE(workspace_bytes >= rq_fused_decode_workspace_bytes(num_seqs, num_q_heads, head_dim, max_seq_len),
                 "workspace too small");
    RQ_CHECK_ARG(workspace != nullptr && ((uintptr_t)workspace % 16) == 0, "workspace must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    DecodeArgs a{};
    a.q = q;
    a.q_ss = q_stride_seq;
    a.q_sh = q_stride_head;
    a.cache = kv_cache;
    a.stride_block = stride_block;
    a.stride_token = stride_token;
    a.block_size = block_size;
    a.H = num_kv_heads;
    a.G = num_q_heads / num_kv_heads;
    a.HQ = num_q_heads;
    a.bt = block_table;
    a.bt_ss = bt_stride_seq;
    a.max_blocks = max_blocks;
    a.seq_lens = seq_lens;
    a.kc = k_centroids;
    a.vc = v_centroids;
    a.nkc = n_k_centroids;
    a.nvc = n_v_centroids;
    a.R = rotation;
    a.rot_block = rot_block;
    a.score_scale = sm_scale * kLog2e;
    {
        const DecodeWorkspace W(num_seqs, num_q_heads, std::max<int64_t>(max_seq_len, 1));
        uint8_t *base = reinterpret_cast<uint8_t *>(workspace);
        a.part_acc = reinterpret_cast<float *>(base + W.part_acc);
        a.part_ml = reinterpret_cast<float *>(base + W.part_ml);
        a.qops = reinterpret_cast<uint32_t *>(base + W.qops);
        a.descs = reinterpret_cast<TileDesc *>(base + W.descs);
        a.tile_prefix = reinterpret_cast<int *>(base + W.tile_prefix);
        a.n_tiles_total = reinterpret_cast<int *>(base + W.n_tiles);
        a.split_m = reinterpret_cast<uint64_t *>(base + W.n_tiles + 8);
    }
    a.num_blocks = num_blocks;
    a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
    a.hpw = 1;
    for (int d = std::min(a.H, kMaxWaves); d >= 1; --d)
        if (a.H % d == 0) {
            a.hpw = d;
            break;
        }
    // 4-bit V: the 16-entry lookups need more registers than 128 (no cap: 140-150 VGPRs,
    // one 8-wave workgroup per CU) or spill at 128; four-head workgroups fit three per
    // CU instead (config-1 shape, mean per call: V4/K4 143.8 -> 130.3 us, V4/K3 122.4 ->
    // 115.2; 3-bit V keeps eight heads: 88.5 against 100.9 us at four).
    if (n_v_centroids == 16 && a.hpw == 8) a.hpw = 4;
    // token stride in a stage: 128 bytes per head, unpadded (swizzled) for one or two heads
    // per workgroup in the nibble layout; else the index runs plus a 16-byte skew
    a.tok_stride = (a.hpw <= 2 && !dense3) ? 128 * a.hpw : 2 * SlotLayout(num_kv_heads, head_dim, dense3).ib * a.hpw + 16;
    a.stage_bytes = kTile * a.tok_stride + 2 * a.hpw * kTile * 4;
    a.max_len = num_blocks > 0 ? (int)std::min<int64_t>(max_blocks * block_size, max_seq_len) : 0;
    a.out = out;
    a.o_ss = out_stride_seq;
    a.o_sh = out_stride_head;
    a.grid_w = 1;
    a.split_c = 1;
    a.wt[0] = a.wt[1] = a.wt[2] = a.wt[3] = 1;
    a.split_r = UINT64_MAX;
    // the stages, the descriptor ring, the query slot and the two codebooks (the
    // kernel variant of this hpw and layout places them the same way)
    const size_t lds = (size_t)decode_stages(a.hpw, dense3) * a.stage_bytes +
                       (size_t)decode_ring(a.hpw, dense3) * sizeof(TileDesc) + (size_t)a.hpw * a.G * 256 + 128;
    int kb = n_k_centroids == 8 ? 3 : 4, vb = n_v_centroids == 8 ? 3 : 4;
    if (a.max_len > 0) {
        if (dtype == RQ_DTYPE_BF16) launch_decode_bits<RQ_DTYPE_BF16>(a, lds, kb, vb, dense3, st, true, {});
        else launch_decode_bits<RQ_DTYPE_F16>(a, lds, kb, vb, dense3, st, true, {});
        // Descriptor workgroups per sequence (y >= 1): enough that each thread writes at
        // most two steps of four tokens of the longest sequence (a fixed three made the
        // prep kernel of a 131072-token sequence take ~49 us).
        const int pthreads = 64 * std::max(4, std::min(a.H, kMaxWaves));
        const int ny = std::min(64, std::max(3, (a.max_len + 8 * pthreads - 1) / (8 * pthreads)));
        const dim3 pgrid((unsigned)num_seqs, (unsigned)(1 + ny)), pblock(pthreads);
        // query staging sized by the waves launched (it bounds how many workgroups a CU holds)
        const size_t plds = (size_t)(pthreads / 64) * 16 * kD * sizeof(uint16_t);
        if (dtype == RQ_DTYPE_BF16) hipLaunchKernelGGL(decode_prep_kernel<RQ_DTYPE_BF16>, pgrid, pblock, plds, st, a);
        else hipLaunchKernelGGL(decode_prep_kernel<RQ_DTYPE_F16>, pgrid, pblock, plds, st, a);
        int rc = check_launch("decode_prep_kernel");
        if (rc) return rc;
        if (dtype == RQ_DTYPE_BF16) launch_decode_bits<RQ_DTYPE_BF16>(a, lds, kb, vb, dense3, st, false, ev);
        else launch_decode_bits<RQ_DTYPE_F16>(a, lds, kb, vb, dense3, st, false, ev);
        rc = check_launch("decode_kernel");
        if (rc) return rc;
    }
    // One wave per (sequence, query head): four per workgroup, or one when the batch has
    // few (sequence, head) pairs, so that they spread over all CUs.
    const int mw = num_seqs * (int64_t)num_q_heads >= 4LL * device_cus() ? 4 : 1;
    // Few pairs whose sequences span many decode workgroups each (at least 8 on
    // average: a tensor-parallel slice, a small batch of long contexts): four waves
    // per pair, each taking every fourth segment pass.
    const bool split = mw == 1 && a.grid_w >= 8 * num_seqs;
    dim3 mgrid(split ? num_q_heads : (num_q_heads + mw - 1) / mw, (unsigned)num_seqs), mblock(64 * (split ? 4 : mw));
    // 32-segment passes when a sequence may span many decode workgroups (very long
    // contexts), or when all merge waves fit at once at the lower occupancy
    // (3 per SIMD); otherwise 16 (config 2: 8192 short merges).  Split merges take
    // 16 while the four waves' first passes cover the average sequence's segments.
    const bool wide = split ? a.grid_w >= 48 * num_seqs
                            : a.max_len >= 65536 || num_seqs * (int64_t)num_q_heads <= 12LL * device_cus();
    auto launch_merge = [&](auto dt) {
        constexpr int DT = decltype(dt)::value;
        if (split && wide) hipLaunchKernelGGL((decode_merge_kernel<DT, 32, 4>), mgrid, mblock, 0, st, a);
        else if (split) hipLaunchKernelGGL((decode_merge_kernel<DT, 16, 4>), mgrid, mblock, 0, st, a);
        else if (wide) hipLaunchKernelGGL((decode_merge_kernel<DT, 32, 1>), mgrid, mblock, 0, st, a);
        else hipLaunchKernelGGL((decode_merge_kernel<DT, 16, 1>), mgrid, mblock, 0, st, a);
    };
    if (dtype == RQ_DTYPE_BF16) launch_merge(std::integral_constant<int, RQ_DTYPE_BF16>{});
    else launch_merge(std::integral_constant<int, RQ_DTYPE_F16>{});
    return check_launch("decode_merge_kernel");
}
