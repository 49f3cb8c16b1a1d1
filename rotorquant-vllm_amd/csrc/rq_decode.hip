// Fused paged decode attention over the packed RotorQuant cache (gfx950).
//
// Replaces fused_paged_rq_decode (src/rotorquant_vllm/triton/fused_paged_rq_decode.py:214-312,
// kernel :32-206).  Same mathematics -- attention in the rotated space, with
// q_rot = bf16(q R^T), K/V = centroid[idx] * norm, exp2 online softmax, and
// out = bf16(bf16(out_rot) R) -- organised for CDNA4 in three launches:
//
//   * decode_prep_kernel: per sequence, the fp16 Q^T MFMA operand of every kv
//     head and one descriptor per 32-token tile (slot offsets from the block
//     table);
//   * decode_kernel: persistent; the tiles of the whole batch are split into
//     equal contiguous ranges, one per resident workgroup.  A workgroup holds
//     one wave per kv head, so each token's K/V bytes are read once and shared
//     by all GQA query heads.  Tiles are copied global -> LDS two ahead;
//     Q K^T and P V run on v_mfma_f32_16x16x32_f16 with the GQA group
//     (<= 16 query heads) as the 16-wide N side; nibble -> fp16 centroid
//     lookups are register v_perm_b32 table lookups and the K/V norms are
//     applied to the scores and to P.  Each sequence segment of a range ends
//     in an (m, l, acc) partial;
//   * decode_merge_kernel: log-sum-exp over a sequence's partials, rounding
//     and the rotation back by R.
//
// MFMA operand layout used below (16x16x32, wave64, lane l, g = l / 16):
//   A (16 x 32): lane holds row l % 16, k = 8g .. 8g+7   (4 dwords of 2 x 16-bit)
//   B (32 x 16): lane holds col l % 16, k = 8g .. 8g+7
//   C (16 x 16): lane holds col l % 16, rows 4g .. 4g+3  (4 floats)
//
// S^T = K Q^T per 16-token group j (A = K: row = token 16j + l%16, k = head
// dims; B = Q^T: col = query head).  Lane (g, q) then holds scores of tokens
// {4g + i} (j = 0) and {16 + 4g + i} (j = 1) for query head q, which is
// exactly the k-group order used for O^T = V^T P^T (A = V^T: row = a head dim,
// k = those 8 tokens; B = P^T: col = query head): no cross-lane movement of P.
#include <algorithm>
#include <mutex>

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

// Centroids (fp32, 16-byte aligned, n = 8 or 16): uniform vector loads issued
// together (entries past n read as zero).
struct Centroids {
    float4 v4[4];
};
__device__ __forceinline__ Centroids load_centroids(const float *c, int n) {
    const float4 *c4 = reinterpret_cast<const float4 *>(c);
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    return Centroids{{c4[0], c4[1], n > 8 ? c4[2] : z, n > 8 ? c4[3] : z}};
}

// Centroids -> 16-bit table split in low / high bytes.
template <int DT>
__device__ __forceinline__ Table16 make_table(const Centroids &cv) {
    const float4 *v4 = cv.v4;
    Table16 t;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float e[4] = {v4[w].x, v4[w].y, v4[w].z, v4[w].w};
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t bits = Elem<DT>::from_f32(e[i]);
            lo |= (bits & 0xffu) << (8 * i);
            hi |= (bits >> 8) << (8 * i);
        }
        t.lo[w] = lo;
        t.hi[w] = hi;
    }
    return t;
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

typedef __attribute__((ext_vector_type(2))) int i32x2;
// ds_read_b64_tr_b8 (gfx950): per 16 lanes, lanes 2i and 2i + 1 name the two 8-byte
// halves of row i of an 8 x 16 byte block, and lane c receives byte c of rows 0..7
// (row i in byte i).  p: an LDS address, 8-byte aligned.
__device__ __forceinline__ i32x2 ds_read_tr8(const uint8_t *p) {
    typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2 *)(p));
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
    uint32_t *qops;     // [seq][H][16 cols][4 g][4 chunks][4 dwords]: fp16 query operands (cols < G written)
    float *qscale;      // [seq][H][16] score scales
    float *part_acc;    // [slot][HQ][D], slot = workgroup + seq
    float *part_ml;     // [slot][HQ][2]
    void *out;
    int64_t o_ss, o_sh;
};

template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (DT == RQ_DTYPE_BF16) {
        typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
        bf16x2 v = {(__bf16)a, (__bf16)b};
        return __builtin_bit_cast(uint32_t, v);
    } else {
        typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
        f16x2 v = {(_Float16)a, (_Float16)b};
        return __builtin_bit_cast(uint32_t, v);
    }
}

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
// dtype, as the fp16 Q^T MFMA operand: lane (g, col) holds for dim chunk c the
// dims 32g + 8c + {0,2,4,6,1,3,5,7} of query head col (zero for col >= G).  The
// rounded q_rot is scaled by 2^qexp (exact) so its largest element sits in
// [2^14, 2^15); sc = score_scale * 2^-qexp undoes it on the scores.
// wq: this wave's LDS scratch of G * 128 16-bit values.
template <int DT>
__device__ __forceinline__ void query_operand(const DecodeArgs &a, int64_t seq, int h, uint16_t *wq, u32x4 (&qop)[4],
                                              float &sc) {
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
    float qv[4][8];
    float qmax = 0.f;
    #pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint4 w = col < a.G ? *reinterpret_cast<const uint4 *>(wq + col * kD + 32 * g + 8 * c)
                                  : make_uint4(0, 0, 0, 0);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    #pragma unroll
        for (int i = 0; i < 4; ++i) {
            qv[c][2 * i] = Elem<DT>::to_f32(ws[i] & 0xffffu);
            qv[c][2 * i + 1] = Elem<DT>::to_f32(ws[i] >> 16);
            qmax = fmaxf(qmax, fmaxf(fabsf(qv[c][2 * i]), fabsf(qv[c][2 * i + 1])));
        }
    }
    qmax = rows_max(qmax);
    const int qexp = qmax > 0.f ? 141 - (int)((__float_as_uint(qmax) >> 23) & 0xffu) : 0;  // 14 - floor(log2 qmax)
    sc = a.score_scale * ldexpf(1.f, -qexp);
    #pragma unroll
    for (int c = 0; c < 4; ++c) {
        float e[8];
    #pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = ldexpf(qv[c][i], qexp);
        qop[c].x = pack2<RQ_DTYPE_F16>(e[0], e[2]);
        qop[c].y = pack2<RQ_DTYPE_F16>(e[4], e[6]);
        qop[c].z = pack2<RQ_DTYPE_F16>(e[1], e[3]);
        qop[c].w = pack2<RQ_DTYPE_F16>(e[5], e[7]);
    }
    __builtin_amdgcn_wave_barrier();
}

// s_waitcnt vmcnt(min(n, MAXN)) for a wave-uniform n.
template <int MAXN>
__device__ __forceinline__ void wait_copies_n(int n) {
    if constexpr (MAXN > 0) {
        if (n >= MAXN) wait_copies<MAXN>();
        else wait_copies_n<MAXN - 1>(n);
    } else {
        wait_copies<0>();
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
constexpr int kRing = 4;                                   // descriptors staged ahead in LDS

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
//   * y == 0: the fp16 query operands (and score scales) of every kv head of the
//     sequence, stored per query-head column (256 bytes each, in the order the
//     decode lanes (g, col) read them) so one copy moves a kv head's G columns;
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
            float sc;
            query_operand<DT>(a, seq, h, reinterpret_cast<uint16_t *>(prep_lds) + wave * 16 * kD, qop, sc);
            const int g = lane >> 4, col = lane & 15;
            uint4 *dst = reinterpret_cast<uint4 *>(a.qops + ((seq * a.H + h) * 16 + col) * 64 + g * 16);
            if (col < a.G) {
    #pragma unroll
                for (int c = 0; c < 4; ++c) dst[c] = make_uint4(qop[c].x, qop[c].y, qop[c].z, qop[c].w);
            }
            if (lane < 16) a.qscale[(seq * a.H + h) * 16 + lane] = sc;
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
        int c_lo = 0, c_hi = 0;
        for (int w = 1 + lane; w < r.G; w += 64) {
            const int rs = range_start(r, w);
            c_lo += rs <= prefix ? 1 : 0;
            c_hi += rs <= prefix + n - 1 ? 1 : 0;
        }
        for (int o = 32; o >= 1; o >>= 1) {
            c_lo += __shfl_xor(c_lo, o);
            c_hi += __shfl_xor(c_hi, o);
        }
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

// Decode.  The tiles of all sequences, in order, are split into gridDim.x equal
// contiguous ranges; workgroup w (with blockIdx.z selecting a group of hpw kv
// heads, one wave per head) takes range w, so every workgroup gets the same work
// whatever the sequence lengths.  A range covers one or more sequence segments;
// each segment ends in a partial (m, l, acc) at slot w + seq, which is unique
// because ranges are contiguous and ordered.
//
// Data movement: tile descriptors are copied into an LDS ring four tiles ahead
// and each tile's K/V index runs and norms two tiles ahead, into two stages:
//   stage layout: token t at t * tok_stride: [K idx of the hpw heads | V idx]
//                 then norm rows (2*hpw x 32 fp32): K norms of each head, V norms.
// One copy instruction moves a whole token's K+V index run (8*hpw x 16 B), so
// every request covers whole cache lines.  Iteration t: wait for tile t (tile
// t+1 stays in flight), barrier, read this wave's operands into registers,
// barrier, copy descriptor t+4 and tile t+2, compute tile t from registers.
// Occupancy 4 (128 VGPRs) where the compiler fits the kernel without spilling.
constexpr int decode_waves_per_eu(int kb, int vb, int hpw) { return (kb + vb == 6 || (kb + vb == 7 && hpw != 4)) ? 4 : 1; }

// D3: the cache holds the dense 3-bit index layout (48 index bytes per head).
template <int DT, int KB, int VB, int HPW, bool D3>
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
    const int g = lane >> 4;    // k-group / row-group
    const int col = lane & 15;  // MFMA column (query head inside the GQA group) / row
    const int h0 = blockIdx.z * hpw;
    const int h = h0 + wave;
    const SlotLayout SL(a.H, kD, D3);
    constexpr int IB = D3 ? 48 : 64;  // index bytes per head
    constexpr bool kTrV = !D3 && HPW > 0;  // V index bytes by transposing LDS reads
    const int TS = HPW > 0 ? 2 * IB * HPW + 16 : a.tok_stride;
    const int norm_off = kTile * TS;
    const int stage_bytes = HPW > 0 ? kTile * TS + 2 * HPW * kTile * 4 : a.stage_bytes;
    const int tl = lane & 31;  // token of this lane in a tile (slot base, norm copy)

    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t *const stage0 = lds;
    uint8_t *const stage1 = lds + stage_bytes;
    const TileDesc *const ring = reinterpret_cast<const TileDesc *>(lds + 2 * stage_bytes);
    // Query operand slot: per wave, its kv head's G columns (256 bytes each), then
    // the score scales of the hpw kv heads (16 floats each).
    const int G = a.G;
    uint8_t *const qarea = lds + 2 * stage_bytes + kRing * sizeof(TileDesc);
    const float *const scarea = reinterpret_cast<const float *>(qarea + hpw * G * 256);

    // Descriptor of local tile i -> ring slot i % kRing (wave 0, one copy).
    auto issue_desc = [&](int i) {
        if (wave == 0 && lane < kDescPieces)
            copy16(reinterpret_cast<const uint8_t *>(a.descs + k0 + i), 16 * lane, lds_addr(reinterpret_cast<const uint8_t *>(ring + i % kRing)));
    };
    // Copies of local tile i into stage sb.  Per wave and full tile: kTile / hpw
    // token copies and one norm copy.
    auto issue = [&](int i, const uint8_t *sb) {
        const TileDesc &d = ring[i % kRing];
        const int valid = __builtin_amdgcn_readfirstlane(d.valid);
        const uint64_t base = d.off[lane_now() & 31];
        const uint32_t dst = lds_addr(sb);
        constexpr int PH = IB / 16;  // 16-byte pieces per head
        const uint32_t kv_src = lane < PH * hpw ? (uint32_t)(SL.k_idx + IB * h0 + 16 * lane)
                                                : (uint32_t)(SL.v_idx + IB * h0 + 16 * (lane - PH * hpw));
        for (int tt = wave; tt < valid; tt += hpw) {
            const uint8_t *tok = a.cache + readlane64(base, tt);  // uniform slot address
            if (lane < 2 * PH * hpw) copy16(tok, kv_src, dst + tt * TS);
        }
        if constexpr (HPW > 0) {
            // Norms in 16-byte pieces: a token's K norms and V norms of the hpw heads
            // are NP pieces; one copy covers TPI tokens (waves 0 .. kTile/TPI - 1).
            // Lane l takes token slot q' = l / NP, piece l % NP, where slot q' holds
            // token 4 (q' % (TPI/4)) + q' / (TPI/4) of the copy's token range: the
            // norms of tokens 4g + i (fixed i) then land 16 NP g bytes apart (distinct
            // banks) and tokens i, i+1, ... 256 bytes apart.
            constexpr int NP = HPW / 2, TPI = 64 / NP;
            if (wave < kTile / TPI) {
                const uint32_t l = lane_now();  // lane-derived values rebuilt here, not kept live
                const int qs = l / NP, p = l % NP;
                const int tt = wave * TPI + 4 * (qs % (TPI / 4)) + qs / (TPI / 4);
                const uint32_t src = p < NP / 2 ? (uint32_t)(SL.k_norm + 4 * h0 + 16 * p)
                                                : (uint32_t)(SL.v_norm + 4 * h0 + 16 * (p - NP / 2));
                if (tt < valid) copy16v(a.cache + d.off[tt] + src, dst + norm_off + 1024 * wave);
            }
        } else {
            // norm rows 2*wave, 2*wave+1 (row j < hpw: K norm of head h0+j, else V norm of head h0+j-hpw)
            const int nrow = 2 * wave + (lane >> 5);
            const uint32_t norm_src = nrow < hpw ? (uint32_t)(SL.k_norm + 4 * (h0 + nrow))
                                                 : (uint32_t)(SL.v_norm + 4 * (h0 + nrow - hpw));
            if (tl < valid) copy4(a.cache + base + norm_src, dst + norm_off + 256 * wave);
        }
    };

    // Query operand and score scales of sequence s -> the query slot (each wave its
    // own kv head): ceil(G / 4) 16-byte copies and one 4-byte copy per wave.
    auto issue_q = [&](int s) {
        const uint8_t *src = reinterpret_cast<const uint8_t *>(a.qops) + ((int64_t)s * a.H + h) * 16 * 256;
        const uint32_t dst = lds_addr(qarea + wave * G * 256);
        const uint32_t l16 = 16u * lane_now();
        for (int j = 0; j < G * 256; j += 1024)
            if (j + l16 < (uint32_t)(G * 256)) copy16(src, j + l16, dst + j);
        if (l16 < 256)
            copy4s(reinterpret_cast<const uint8_t *>(a.qscale + ((int64_t)s * a.H + h) * 16), l16 >> 2,
                   lds_addr(reinterpret_cast<const uint8_t *>(scarea + wave * 16)));
    };

    // The centroid loads are compiler-visible: issued before the descriptor copies
    // and covered by their wait, so no wait of the compiler's for them lands after
    // the first tile copies (it would wait for those too).
    const Centroids ck = load_centroids(a.kc, a.nkc), cv = load_centroids(a.vc, a.nvc);
    for (int i = 0; i < min(nt, kRing); ++i) issue_desc(i);
    wait_copies<0>();
    __syncthreads();

    const Table16 tk = make_table<RQ_DTYPE_F16>(ck);
    const Table16 tv = make_table<RQ_DTYPE_F16>(cv);

    // Per-segment state.  No compiler-visible global load is issued inside the tile
    // loop: the compiler does not count the copies, so a wait it inserted for a load
    // of its own would wait for every copy in flight and stall the pipeline.  The
    // query operand therefore arrives by copy, in the same stream as the tiles.
    int seq = -1;
    u32x4 qop[4];
    float sc;
    f32x4 acc[8];
    float m_run, l_run;
    int e_run;      // every V norm of the segment so far is < 2^e_run
    float lim;      // 2^e_run
    auto begin_segment = [&]() {
        const uint32_t ln = lane_now(), lc = ln & 15;  // rebuilt here, not kept live across the loop
        const uint4 *src = reinterpret_cast<const uint4 *>(qarea + wave * G * 256 + lc * 256 + (ln >> 4) * 64);
    #pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 v = (int)lc < G ? src[c] : make_uint4(0, 0, 0, 0);
            qop[c] = u32x4{v.x, v.y, v.z, v.w};
        }
        sc = (int)lc < G ? scarea[wave * 16 + lc] : 1.f;  // columns >= G: zero queries, any positive scale
    #pragma unroll
        for (int m = 0; m < 8; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
        m_run = -INFINITY;  // running max (log2 domain) for query head `col`
        l_run = 0.f;        // this lane's partial sum of p' = p * 2^-e_run
        // P operand = p' * v_norm = p * v_norm * 2^-e_run <= 2^8 (fp16).  acc and l_run
        // carry the factor 2^-e_run, so the partial is (m_run + e_run, l_run, acc).
        // Starting at 2^-64 keeps p' <= 2^72 and l_run finite for tiny norms.
        e_run = -64;
        lim = 0x1p-64f;
    };
    // Partial of the current segment -> slot w + seq.  Addresses are a uniform
    // 64-bit base plus a 32-bit lane offset computed here (a hoisted 64-bit per-lane
    // address would be spilled, and its reload would wait for the copies in flight).
    auto end_segment = [&]() {
        const float lsum = rows_sum(l_run);
        if (col < a.G) {
            const int64_t slot = (int64_t)(w + seq) * a.HQ + h * a.G;  // uniform: query head h*G of the slot
            uint8_t *pa = reinterpret_cast<uint8_t *>(a.part_acc + slot * kD);
            uint8_t *pm = reinterpret_cast<uint8_t *>(a.part_ml + slot * 2);
            const uint32_t ln = lane_now();
            if constexpr (!kTrV) {
                // acc[m][i] = O[col][8 * (4g + i) + m] relative to 2^(m_run + e_run)
                const uint32_t lo_off = ((ln & 15) * kD + 32 * (ln >> 4)) * 4;
    #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float4 lo = make_float4(acc[0][i], acc[1][i], acc[2][i], acc[3][i]);
                    float4 hi = make_float4(acc[4][i], acc[5][i], acc[6][i], acc[7][i]);
                    float4 *dst = reinterpret_cast<float4 *>(pa + lo_off + 32 * i);
                    dst[0] = lo;
                    dst[1] = hi;
                }
            } else {
                // acc[2r + e][i] = O[col][32r + 8g + 2i + e] relative to 2^(m_run + e_run)
                const uint32_t lo_off = ((ln & 15) * kD + 8 * (ln >> 4)) * 4;
    #pragma unroll
                for (int i = 0; i < 4; ++i)
    #pragma unroll
                    for (int r = 0; r < 4; ++r)
                        *reinterpret_cast<float2 *>(pa + lo_off + 4 * (32 * r + 2 * i)) =
                            make_float2(acc[2 * r][i], acc[2 * r + 1][i]);
            }
            if (g == 0) *reinterpret_cast<float2 *>(pm + 8u * (lane_now() & 15)) = make_float2(m_run + (float)e_run, lsum);
        }
    };
    // The query slot holds the operand of the segment starting at local tile q_upto;
    // the next one is copied once that segment has begun (its operand is then in
    // registers), before the tile copies of the same iteration, so the wait for the
    // tile that starts the new segment also covers it.
    int q_upto = 0;
    issue_q(__builtin_amdgcn_readfirstlane(ring[0].seq));
    issue(0, stage0);
    if (nt > 1) issue(1, stage1);

    for (int t = 0; t < nt; ++t) {
        const uint8_t *const sb = (t & 1) ? stage1 : stage0;
        // Tile t landed?  Issued after its copies, and allowed to stay in flight:
        // this wave's copies of tile t+1 (iteration t-1) and descriptor t+3 (wave 0,
        // iteration t-1; the prologue issues descriptors 0..3 before tile 0).  The
        // query operand copies of an iteration precede both.
        if (HPW > 0 && t + 1 < nt) {
            constexpr int HP = HPW > 0 ? HPW : 8, TPI = 128 / HP;
            const int v1 = __builtin_amdgcn_readfirstlane(ring[(t + 1) % kRing].valid);
            // token copies tt = wave, wave + HPW, ... < v1; a norm copy on the waves
            // whose token range [wave * TPI, +TPI) starts below v1
            const int n = (v1 > wave ? (v1 - wave + HP - 1) / HP : 0) + (wave < kTile / TPI && wave * TPI < v1 ? 1 : 0) +
                          (wave == 0 && t >= 1 && t + 3 < nt ? 1 : 0);
            wait_copies_n<kTile / HP + 2>(n);
        } else {
            wait_copies<0>();
        }
        __syncthreads();

        const int tseq = __builtin_amdgcn_readfirstlane(ring[t % kRing].seq);
        const int valid = __builtin_amdgcn_readfirstlane(ring[t % kRing].valid);
        if (tseq != seq) {  // a new sequence starts at this tile
            if (seq >= 0) end_segment();
            seq = tseq;
            begin_segment();
        }
        // ---- this wave's operands of the tile ------------------------------------
        // token col, K dims 32g .. 32g+31 (16 nibble bytes, or the 12-byte dense group g)
        const uint8_t *kb = sb + col * TS + IB * wave + (D3 ? 12 : 16) * g;
        // V index bytes of the lane's 8 tokens 4g + k, 16 + 4g + k (k < 4), transposed:
        // Ga[r] = byte j of tokens 4g .. 4g+3 (byte k = token 4g + k), Gb[r] = byte j of
        // tokens 16+4g .. 16+4g+3.
        //   nibbles, 8 or 4 heads per workgroup: j = 16r + col (dims 32r + 2 col, +1) by
        //     ds_read_b64_tr_b8, which transposes, per 16 lanes, an 8 x 16 byte block:
        //     lanes 2i and 2i + 1 give the two 8-byte halves of row i (token i of the lane
        //     group), and lane c gets byte c of every row;
        //   otherwise j = r of the nibble dword col (dims 8 col + 2r, +1), or dense: of
        //     dword min(col % 4, 2) of group col / 4 (position 3 is assembled from the
        //     quad's other three lanes), read per token and byte-transposed in registers
        //     (the generic-head variant has no VGPRs to spare for the other form).
        uint32_t vw[8], Ga[4], Gb[4];
        const uint8_t *nb = sb + norm_off + 128 * wave + 16 * g;               // K norms of tokens 4g..4g+3
        uint4 kw0, kw1;
        if constexpr (D3) {
            const uint32_t *k0p = reinterpret_cast<const uint32_t *>(kb);
            const uint32_t *k1p = reinterpret_cast<const uint32_t *>(kb + 16 * TS);
            kw0 = make_uint4(k0p[0], k0p[1], k0p[2], 0u);
            kw1 = make_uint4(k1p[0], k1p[1], k1p[2], 0u);
        } else {
            kw0 = *reinterpret_cast<const uint4 *>(kb);
            kw1 = *reinterpret_cast<const uint4 *>(kb + 16 * TS);
        }
        if constexpr (!kTrV) {
            const uint8_t *vb = sb + 4 * g * TS + IB * hpw + IB * wave +
                                (D3 ? 12 * (col >> 2) + 4 * min(col & 3, 2) : 4 * col);
    #pragma unroll
            for (int i = 0; i < 8; ++i) vw[i] = *reinterpret_cast<const uint32_t *>(vb + (i < 4 ? i : 12 + i) * TS);
        } else {
            const int row = col >> 1;  // token 4g + row (row < 4) or 12 + 4g + row
            const uint8_t *vr = sb + (row < 4 ? 4 * g + row : 12 + 4 * g + row) * TS + IB * hpw + IB * wave + 8 * (col & 1);
    #pragma unroll
            for (int r = 0; r < 4; ++r) {
                const i32x2 t = ds_read_tr8(vr + 16 * r);
                Ga[r] = (uint32_t)t.x;
                Gb[r] = (uint32_t)t.y;
            }
        }
        float4 nk0, nk1, nv0, nv1;
        if constexpr (HPW > 0) {
            // token 4g + i at 256 i + 16 NP q (+1024 for tokens 16.. when TPI = 16),
            // q = g (tokens < 16) or 4 + g (tokens >= 16 when TPI = 32)
            constexpr int NP = HPW / 2, TPI = 64 / NP;
            const float *n0 = reinterpret_cast<const float *>(sb + norm_off + 16 * NP * g + 16 * (wave / 4) + 4 * (wave % 4));
            const int hi = TPI == 16 ? 1024 : 16 * NP * 4;  // tokens 16..31
            const int vo = 16 * (NP / 2);                     // V norms after the K pieces
            auto ld4 = [&](int o) {
                const float *p = reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(n0) + o);
                return make_float4(p[0], p[64], p[128], p[192]);
            };
            nk0 = ld4(0);
            nk1 = ld4(hi);
            nv0 = ld4(vo);
            nv1 = ld4(vo + hi);
        } else {
            nk0 = *reinterpret_cast<const float4 *>(nb);
            nk1 = *reinterpret_cast<const float4 *>(nb + 64);
            nv0 = *reinterpret_cast<const float4 *>(nb + 128 * hpw);
            nv1 = *reinterpret_cast<const float4 *>(nb + 128 * hpw + 64);
        }
        __syncthreads();  // the stage and descriptor slot t are free once every wave holds its operands

        // ---- next query operand, descriptor t+4 and tile t+2 -------------------------
        if (q_upto <= t && t + 1 < nt) {
            const int s1 = __builtin_amdgcn_readfirstlane(ring[(t + 1) % kRing].seq);
            if (s1 != seq) {
                issue_q(s1);
                q_upto = t + 1;
            } else if (t + 2 < nt) {
                const int s2 = __builtin_amdgcn_readfirstlane(ring[(t + 2) % kRing].seq);
                if (s2 != s1) {
                    issue_q(s2);
                    q_upto = t + 2;
                }
            }
        }
        if (t + kRing < nt) issue_desc(t + kRing);
        if (t + 2 < nt) issue(t + 2, sb);

        // ---- tokens past the end were not copied: their stage bytes are stale.  Zero
        // their norms and V indices (a stale nibble >= 8 would look up a NaN in an
        // 8-entry table, and NaN * 0 would reach the accumulator); their scores are
        // masked below.
        float nk[8] = {nk0.x, nk0.y, nk0.z, nk0.w, nk1.x, nk1.y, nk1.z, nk1.w};
        float nv[8] = {nv0.x, nv0.y, nv0.z, nv0.w, nv1.x, nv1.y, nv1.z, nv1.w};
        if (valid < kTile) {
            // (each masking block takes `valid` through an empty asm, so that its
            // compares stay inside the block instead of running for every full tile)
            const int vv = opaque_s(valid);
            const int g4 = 4 * (int)(lane_now() >> 4);  // 4g, rebuilt here (not kept live)
    #pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int tt = i < 4 ? g4 + i : 12 + g4 + i;
                nk[i] = tt < vv ? nk[i] : 0.f;
                nv[i] = tt < vv ? nv[i] : 0.f;
                if constexpr (!kTrV) vw[i] = tt < vv ? vw[i] : 0u;
            }
            if constexpr (kTrV) {
                uint32_t ma = 0, mb = 0;  // bytes of the tokens 4g + k and 16 + 4g + k below valid
    #pragma unroll
                for (int k = 0; k < 4; ++k) {
                    ma |= (g4 + k < vv ? 0xffu : 0u) << (8 * k);
                    mb |= (16 + g4 + k < vv ? 0xffu : 0u) << (8 * k);
                }
    #pragma unroll
                for (int r = 0; r < 4; ++r) {
                    Ga[r] &= ma;
                    Gb[r] &= mb;
                }
            }
        }
        // A V norm at or above 2^e_run (rare after the first tile): raise e_run to the
        // tile's largest norm (over all 32 tokens: the four row groups of the wave)
        // and rescale what carries 2^-e_run.
        const float nvl = fmaxf(fmaxf(fmaxf(nv[0], nv[1]), fmaxf(nv[2], nv[3])), fmaxf(fmaxf(nv[4], nv[5]), fmaxf(nv[6], nv[7])));
        if (__any(nvl >= lim)) {
            const float nvm = rows_max(nvl);
            const int e_tile = (int)((__float_as_uint(nvm) >> 23) & 0xffu) - 126;  // 2^e_tile > max norm
            if (e_tile > e_run) {
                const float f = ldexpf(1.f, e_run - e_tile);
    #pragma unroll
                for (int m = 0; m < 8; ++m) acc[m] *= f;
                l_run *= f;
                e_run = e_tile;
                lim = ldexpf(1.f, e_run);
            }
        }

        // ---- S^T = K Q^T ----------------------------------------------------
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
                s0 = mfma<RQ_DTYPE_F16>(decode_row8_sel<KB>(tk, e0, o0), qop[c], s0);
                s1 = mfma<RQ_DTYPE_F16>(decode_row8_sel<KB>(tk, e1, o1), qop[c], s1);
            }
        } else {
            const uint32_t k0w[4] = {kw0.x, kw0.y, kw0.z, kw0.w};
            const uint32_t k1w[4] = {kw1.x, kw1.y, kw1.z, kw1.w};
    #pragma unroll
            for (int c = 0; c < 4; ++c) {
                s0 = mfma<RQ_DTYPE_F16>(decode_row8<KB>(tk, k0w[c]), qop[c], s0);
                s1 = mfma<RQ_DTYPE_F16>(decode_row8<KB>(tk, k1w[c]), qop[c], s1);
            }
        }
        // ---- scale by K norm, mask, online softmax ---------------------------
        // s = score / sc; the score scale sc > 0 enters the exponent's fma (and the
        // max, which it commutes with).
        float s[8] = {s0.x * nk[0], s0.y * nk[1], s0.z * nk[2], s0.w * nk[3],
                      s1.x * nk[4], s1.y * nk[5], s1.z * nk[6], s1.w * nk[7]};
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
        // than 8 (log2 units).  In between, p = 2^(score - m_run) <= 2^8, so the
        // fp16 P operand (p * v_norm * 2^-e_run <= 2^8) stays in range; acc and l_run
        // are relative to the same m_run, so the result does not depend on when the
        // rescale happens.  The exponent's fma also applies 2^-e_run.
        if (__any(tmax > m_run + 8.f)) {
            const float m_new = fmaxf(m_run, tmax);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // m_run = -inf on the first tile -> 0
    #pragma unroll
            for (int m = 0; m < 8; ++m) acc[m] *= alpha;
            l_run *= alpha;
            m_run = m_new;
        }
        const float mb = -(m_run + (float)e_run);
        float p[8];
    #pragma unroll
        for (int i = 0; i < 8; ++i) {
            p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], sc, mb));  // p * 2^-e_run
            l_run += p[i];
        }
        u32x4 pop;
        pop.x = pack2<RQ_DTYPE_F16>(p[0] * nv[0], p[1] * nv[1]);
        pop.y = pack2<RQ_DTYPE_F16>(p[2] * nv[2], p[3] * nv[3]);
        pop.z = pack2<RQ_DTYPE_F16>(p[4] * nv[4], p[5] * nv[5]);
        pop.w = pack2<RQ_DTYPE_F16>(p[6] * nv[6], p[7] * nv[7]);

        // ---- O^T += V^T P^T ---------------------------------------------------
        // Ga[j], Gb[j]: byte j of the lane's tokens (read transposed above, or here
        // byte-transposed from the tokens' dwords); split nibbles per head dim.
        if constexpr (!kTrV) {
            const uint32_t A01 = perm(vw[1], vw[0], 0x05010400u), B01 = perm(vw[1], vw[0], 0x07030602u);
            const uint32_t A23 = perm(vw[3], vw[2], 0x05010400u), B23 = perm(vw[3], vw[2], 0x07030602u);
            const uint32_t A45 = perm(vw[5], vw[4], 0x05010400u), B45 = perm(vw[5], vw[4], 0x07030602u);
            const uint32_t A67 = perm(vw[7], vw[6], 0x05010400u), B67 = perm(vw[7], vw[6], 0x07030602u);
            Ga[0] = perm(A23, A01, 0x05040100u);
            Ga[1] = perm(A23, A01, 0x07060302u);
            Ga[2] = perm(B23, B01, 0x05040100u);
            Ga[3] = perm(B23, B01, 0x07060302u);
            Gb[0] = perm(A67, A45, 0x05040100u);
            Gb[1] = perm(A67, A45, 0x07060302u);
            Gb[2] = perm(B67, B45, 0x05040100u);
            Gb[3] = perm(B67, B45, 0x07060302u);
        }
        // Index selectors (one index per byte) of the even and the odd dim of byte j.
        // Dense: lanes of positions 0..2 mask their own bytes; the position-3 lane takes
        // the top bits of its quad's A, B and C lanes (same tokens): one form for all
        // lanes, (x >> s1) & m1 | (y >> s2) & m2, with per-lane shifts and masks.
        auto sel = [&](uint32_t G, uint32_t &ev, uint32_t &od) {
            if constexpr (D3) {
                const bool p3 = (col & 3) == 3;
                const uint32_t xe = quad_pick<0x24>(G), xo = quad_pick<0x64>(G), y = quad_pick<0xa4>(G);
                const uint32_t m1 = p3 ? 0x03030303u : 0x07070707u, m2 = p3 ? 0x04040404u : 0u;
                ev = ((xe >> (p3 ? 6 : 0)) & m1) | ((y >> 4) & m2);
                od = ((xo >> (p3 ? 6 : 3)) & m1) | ((y >> 5) & m2);
            } else {
                ev = (G >> 4) & 0x0f0f0f0fu;
                od = G & 0x0f0f0f0fu;
            }
        };
    #pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t ea, oa, eb, ob;
            sel(Ga[j], ea, oa);
            sel(Gb[j], eb, ob);
            uint2 ha = lookup4<VB>(tv, ea), hb = lookup4<VB>(tv, eb);
            uint2 la = lookup4<VB>(tv, oa), lb = lookup4<VB>(tv, ob);
            acc[2 * j] = mfma<RQ_DTYPE_F16>(u32x4{ha.x, ha.y, hb.x, hb.y}, pop, acc[2 * j]);          // even dims
            acc[2 * j + 1] = mfma<RQ_DTYPE_F16>(u32x4{la.x, la.y, lb.x, lb.y}, pop, acc[2 * j + 1]);  // odd dims
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
template <int DT, int kMergePass>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    const int64_t seq = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int hq = blockIdx.x * 4 + wave;
    __shared__ float orot_all[4][kD];
    float *orot = orot_all[wave];
    if (hq >= a.HQ) return;
    // R entries for this lane's two output dims (issued first; independent of the partials)
    float rr[2][4];
    #pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int d = 2 * lane + e;
        const int k0 = (d / a.rot_block) * a.rot_block;
    #pragma unroll
        for (int i = 0; i < 4; ++i) rr[e][i] = i < a.rot_block ? a.R[(k0 + i) * kD + d] : 0.f;
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
    for (int c0 = 0; c0 < nch; c0 += kMergePass) {
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
        const float alpha = __builtin_amdgcn_exp2f(M - Mn);  // -inf - finite -> 0 on the first pass
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

constexpr int kMaxWgPerCu = 4;  // bound on decode workgroups per CU (sizes the partial slots)

// Resident decode workgroups per CU for an LDS size (cached per device and size).
template <int DT, int KB, int VB, int HPW, bool D3>
static int decode_per_cu(const DecodeArgs &a, size_t lds) {
    static int cache[64][8][2] = {};  // [device][entry] = {lds, workgroups per CU}
    int dev = 0;
    (void)hipGetDevice(&dev);
    dev = dev < 0 || dev >= 64 ? 0 : dev;
    for (auto &e : cache[dev])
        if (e[0] == (int)lds && e[1] > 0) return e[1];
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void *>(&decode_kernel<DT, KB, VB, HPW, D3>),
                                                      64 * a.hpw, lds) != hipSuccess || nb <= 0)
        nb = 1;
    nb = std::min(nb, kMaxWgPerCu);
    for (auto &e : cache[dev])
        if (e[1] == 0) {
            e[0] = (int)lds;
            e[1] = nb;
            break;
        }
    return nb;
}

// configure: set the grid and range split only (before the prep kernel, which
// needs them); otherwise launch.
template <int DT, int KB, int VB, int HPW, bool D3>
static void launch_decode_h(DecodeArgs &a, size_t lds, hipStream_t st, bool configure) {
    if (!configure) {
        hipLaunchKernelGGL((decode_kernel<DT, KB, VB, HPW, D3>), dim3((unsigned)a.grid_w, 1, a.H / a.hpw), dim3(64 * a.hpw),
                           lds, st, a);
        return;
    }
    // as many workgroups per kv-head group as are resident at once
    const int per_cu = decode_per_cu<DT, KB, VB, HPW, D3>(a, lds);
    const int groups = a.H / a.hpw;
    a.grid_w = std::max(1, per_cu * device_cus() / groups);
    // rank weights by workgroups per CU (workgroups [r CUs, (r+1) CUs) are
    // dispatched r-th onto each CU)
    static const int kRankWt[5][4] = {{1, 1, 1, 1}, {1, 1, 1, 1}, {65, 35, 35, 35}, {1, 1, 1, 1}, {1, 1, 1, 1}};
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

template <int DT, int KB, int VB, bool D3 = false>
static void launch_decode(DecodeArgs &a, size_t lds, hipStream_t st, bool configure) {
    if (a.hpw == 8) launch_decode_h<DT, KB, VB, 8, D3>(a, lds, st, configure);
    else if (a.hpw == 4) launch_decode_h<DT, KB, VB, 4, D3>(a, lds, st, configure);
    else launch_decode_h<DT, KB, VB, 0, D3>(a, lds, st, configure);
}

template <int DT>
static void launch_decode_bits(DecodeArgs &a, size_t lds, int kb, int vb, bool dense3, hipStream_t st,
                               bool configure) {
    if (dense3) launch_decode<DT, 3, 3, true>(a, lds, st, configure);  // the layout holds 3-bit indices only
    else if (kb == 3 && vb == 3) launch_decode<DT, 3, 3>(a, lds, st, configure);
    else if (kb == 3) launch_decode<DT, 3, 4>(a, lds, st, configure);
    else if (vb == 3) launch_decode<DT, 4, 3>(a, lds, st, configure);
    else launch_decode<DT, 4, 4>(a, lds, st, configure);
}

// Workspace layout (256-byte aligned regions).
struct DecodeWorkspace {
    int64_t part_acc, part_ml, qops, qscale, descs, tile_prefix, n_tiles, total;
    DecodeWorkspace(int64_t num_seqs, int64_t num_q_heads, int64_t max_seq_len) {
        auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
        const int64_t slots = (int64_t)kMaxWgPerCu * device_cus() + num_seqs;
        const int64_t max_tiles = num_seqs * ((max_seq_len + kTile - 1) / kTile);
        part_acc = 0;
        part_ml = al(part_acc + slots * num_q_heads * kD * 4);
        qops = al(part_ml + slots * num_q_heads * 2 * 4);
        qscale = al(qops + num_seqs * num_q_heads * 64 * 16 * 4);  // kv heads <= query heads
        descs = al(qscale + num_seqs * num_q_heads * 16 * 4);
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
                             int64_t workspace_bytes, void *stream);

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
                             int64_t workspace_bytes, void *stream) {
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
        a.qscale = reinterpret_cast<float *>(base + W.qscale);
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
    a.tok_stride = 2 * SlotLayout(num_kv_heads, head_dim, dense3).ib * a.hpw + 16;
    a.stage_bytes = kTile * a.tok_stride + 2 * a.hpw * kTile * 4;
    a.max_len = num_blocks > 0 ? (int)std::min<int64_t>(max_blocks * block_size, max_seq_len) : 0;
    a.out = out;
    a.o_ss = out_stride_seq;
    a.o_sh = out_stride_head;
    a.grid_w = 1;
    a.split_c = 1;
    a.wt[0] = a.wt[1] = a.wt[2] = a.wt[3] = 1;
    a.split_r = UINT64_MAX;
    const size_t lds = 2 * (size_t)a.stage_bytes + kRing * sizeof(TileDesc) + (size_t)a.hpw * (a.G * 256 + 64);
    int kb = n_k_centroids == 8 ? 3 : 4, vb = n_v_centroids == 8 ? 3 : 4;
    if (a.max_len > 0) {
        if (dtype == RQ_DTYPE_BF16) launch_decode_bits<RQ_DTYPE_BF16>(a, lds, kb, vb, dense3, st, true);
        else launch_decode_bits<RQ_DTYPE_F16>(a, lds, kb, vb, dense3, st, true);
        // Descriptor workgroups per sequence (y >= 1): enough that each thread writes at
        // most two steps of four tokens of the longest sequence (a fixed three made the
        // prep kernel of a 131072-token sequence take ~49 us).
        const int pthreads = 64 * std::min(a.H, kMaxWaves);
        const int ny = std::min(64, std::max(3, (a.max_len + 8 * pthreads - 1) / (8 * pthreads)));
        const dim3 pgrid((unsigned)num_seqs, (unsigned)(1 + ny)), pblock(pthreads);
        // query staging sized by the waves launched (it bounds how many workgroups a CU holds)
        const size_t plds = (size_t)(pthreads / 64) * 16 * kD * sizeof(uint16_t);
        if (dtype == RQ_DTYPE_BF16) hipLaunchKernelGGL(decode_prep_kernel<RQ_DTYPE_BF16>, pgrid, pblock, plds, st, a);
        else hipLaunchKernelGGL(decode_prep_kernel<RQ_DTYPE_F16>, pgrid, pblock, plds, st, a);
        int rc = check_launch("decode_prep_kernel");
        if (rc) return rc;
        if (dtype == RQ_DTYPE_BF16) launch_decode_bits<RQ_DTYPE_BF16>(a, lds, kb, vb, dense3, st, false);
        else launch_decode_bits<RQ_DTYPE_F16>(a, lds, kb, vb, dense3, st, false);
        rc = check_launch("decode_kernel");
        if (rc) return rc;
    }
    dim3 mgrid((num_q_heads + 3) / 4, (unsigned)num_seqs);
    // 32-segment passes when a sequence may span many decode workgroups (very long
    // contexts), or when all merge waves fit at once at the lower occupancy
    // (3 per SIMD); otherwise 16 (config 2: 8192 short merges).
    const bool wide = a.max_len >= 65536 || num_seqs * (int64_t)num_q_heads <= 12LL * device_cus();
    if (dtype == RQ_DTYPE_BF16) {
        if (wide) hipLaunchKernelGGL((decode_merge_kernel<RQ_DTYPE_BF16, 32>), mgrid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((decode_merge_kernel<RQ_DTYPE_BF16, 16>), mgrid, dim3(256), 0, st, a);
    } else {
        if (wide) hipLaunchKernelGGL((decode_merge_kernel<RQ_DTYPE_F16, 32>), mgrid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((decode_merge_kernel<RQ_DTYPE_F16, 16>), mgrid, dim3(256), 0, st, a);
    }
    return check_launch("decode_merge_kernel");
}
