// Attention of new query tokens over the packed RotorQuant cache, with K and V
// dequantized to the q dtype inside the kernel (gfx950): the backend's
// non-fused path in one launch.
//
// Replaces, in RQAttentionImpl.forward's non-fused path
// (src/rotorquant_vllm/vllm/rq_backend.py:937-1036), the q pre-rotation
// (:939-941, :981), _decompress_cache_paged (:737-852), vLLM's
// flash_attn_varlen_func over the decompressed pages (:996-1030) and the
// back-rotation (:1032-1034).  Arithmetic:
//   * q_rot = q R^T rounded to the q dtype (fma chain over R's diagonal block);
//   * K, V = dtype(centroid * norm): the values rq_decompress writes
//     (isoquant_decompress.py:15-60), never stored to memory;
//   * S = q_rot K^T on the 16-bit MFMA (exact products, fp32 sums), scaled by
//     sm_scale * log2(e); online softmax in base 2;
//   * P V on the fp16 MFMA with P' = p 2^(e_tile - e_run) and
//     V' = V 2^-e_tile (exact for bf16 / fp16 V in fp16 range), the row sum an
//     extra MFMA row -- the P V step of rq_prefill.hip;
//   * out_rot rounded to the q dtype, out = out_rot R rounded again.
// Query i of sequence b sits at position seq_lens[b] - q_len_b + i.  Causal:
// it sees the keys at positions <= its own (flash attention's bottom-right
// aligned mask with seqused_k); otherwise all seq_lens[b] keys.
//
// One workgroup per (query block, kv head, sequence); its waves are (query
// head of the GQA group, 16-position group), as in rq_prefill.hip.  The
// workgroup decodes each 64-key tile of its (sequence, kv head) from the
// packed slots into a double-buffered LDS tile (K rows in the q dtype, fp16
// V'^T rows): while tile t is computed, tile t+1's packed bytes are copied
// cache -> LDS staging with direct global -> LDS copies, and decoded into the
// other buffer after it.  No workspace, no decompressed copy of the cache.
//
// MFMA v_mfma_f32_16x16x32_{bf16,f16} for S^T = K Q^T (wave64, lane l,
// g = l / 16, col = l % 16), four k-steps of 32 head dims:
//   A (16 keys x 32 dims): lane holds key 16b + col, dims 32s + 8g .. +7;
//   B (32 dims x 16 positions): lane holds position col, the same dims;
//   C: lane (g, col) holds position col's scores of keys 16b + 4g + i.
#include <algorithm>

#include "rq_attn_tile.h"

namespace rq {

namespace {

constexpr int kD = kAttnD;
constexpr int kKT = kAttnKT;
constexpr int kPQ = kAttnPQ;

// LDS, per workgroup:
//   two tile buffers: K rows (64 keys x 256 bytes in the q dtype, 16-byte piece
//     c = dims 8c .. 8c+7 of key r, in the order e0 e2 e4 e6 e1 e3 e5 e7, at
//     r * 256 + 16 * (c ^ (r & 15)): the 16 keys one MFMA operand read touches
//     hit 16 distinct piece slots), then V'^T (vt_piece);
//   staging: the next tile's packed bytes as copied from the cache -- K index
//     dwords [key][16], V index dwords [key][16], K norms [key], V norms [key];
//   slot offsets of the keys of the tile staged next.
constexpr int kTK = 0;
constexpr int kTVt = kKT * kD * 2;
constexpr int kTileBytes = kTVt + kD * kKT * 2;
__host__ __device__ constexpr int kt_piece(int r, int c) { return r * 256 + 16 * (c ^ (r & 15)); }
constexpr int kSKi = 2 * kTileBytes;
constexpr int kSVi = kSKi + kKT * 64;
constexpr int kSKn = kSVi + kKT * 64;
constexpr int kSVn = kSKn + kKT * 4;
constexpr int kSOff = kSVn + kKT * 4;
constexpr int kLdsBytes = kSOff + kKT * 8;
constexpr int kCopies = 34;  // wave-wide 4-byte copies per tile: 16 + 16 index, 2 norm

// Decode work of one tile: 256 K items (key quad, dword) and 256 V items.
constexpr int kItems = 512;
constexpr int kMinWaves = 4;  // so that a thread has at most 2 items
constexpr int kMaxWaves = 8;  // GQA groups above 8 heads are split over workgroups

struct AttnArgs {
    const void *q;
    int64_t q_st, q_sh;
    const int32_t *cu_q;
    const uint8_t *cache;
    int64_t stride_block, stride_token;
    int block_size, bs_shift;
    int64_t num_blocks;
    int H, G;
    int dense3;  // dense 3-bit index layout of the cache
    int hsplit;  // workgroups per kv head: each takes G / hsplit query heads
    const int32_t *bt;
    int64_t bt_ss, max_blocks;
    const int32_t *seq_lens;
    const float *kc, *vc;
    int nkc, nvc;
    const float *R;
    int rot_block;
    int causal;
    float score_scale;  // sm_scale * log2(e)
    int qb;             // query positions per workgroup (= 16 * position groups)
    int npg;            // position groups per workgroup
    int ncomp;          // waves that compute (query head, position group); the rest only decode tiles
    void *out;
    int64_t o_st, o_sh;
};

template <int DT>
__global__ __launch_bounds__(64 * kMaxWaves) void paged_attn_kernel(AttnArgs a) {
    int qblk, hy;
    int64_t seq;
    attn_work_item(qblk, hy, seq);
    const int h = hy / a.hsplit, hpart = hy - h * a.hsplit;
    const int q0 = a.cu_q[seq], q1 = a.cu_q[seq + 1];
    const int T = q1 - q0;
    const int L = a.seq_lens[seq];
    const int pos_base = L - T;  // position of query 0
    if (qblk * a.qb >= T || T <= 0) return;
    // keys the block table can address
    const int L_eff = (int)std::min<int64_t>((int64_t)max(L, 0), a.max_blocks * a.block_size);

    const int tid = threadIdx.x, nthr = blockDim.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int nwaves = nthr >> 6;
    const int g = lane >> 4, col = lane & 15;
    const int gw = a.G / a.hsplit;                   // query heads of this workgroup
    const int gh = hpart * gw + wave / a.npg;        // query head inside the GQA group
    const int pg = wave % a.npg;                     // 16-position group
    const int hq = h * a.G + gh;
    const int i0 = qblk * a.qb + pg * kPQ;  // first query index of this wave
    const bool wave_active = wave < a.ncomp && i0 < T;
    const int my_pos = pos_base + i0 + col;
    // V'^T pieces of this lane (dim col, pieces g and 4 + g)
    const int voff0 = vt_piece(col, g), voff1 = vt_piece(col, 4 + g);

    // Keys [0, kv_end) may be visible to some query of the workgroup.
    const int last_i = min(T, (qblk + 1) * a.qb) - 1;
    const int kv_end = a.causal ? min(L_eff, pos_base + last_i + 1) : L_eff;
    const int n_tiles = kv_end > 0 ? (kv_end + kKT - 1) / kKT : 0;

    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float ktab[16], vtab[16];
    if (tid < 16) {
        ktab[tid] = tid < a.nkc ? a.kc[tid] : 0.f;
        vtab[tid] = tid < a.nvc ? a.vc[tid] : 0.f;
    }
    const SlotLayout SL(a.H, kD, a.dense3 != 0);
    const uint32_t lds0 = lds_addr(lds);
    uint64_t *soff = reinterpret_cast<uint64_t *>(lds + kSOff);

    // ---- tile pipeline ------------------------------------------------------
    // Wave 0 turns tile t's block-table entries into slot offsets (one key per
    // lane: issue_bt loads the entry, put_offsets stores the offset); every wave
    // then copies its share of the tile's packed bytes cache -> staging with
    // direct global -> LDS copies (stage); after they land, every thread decodes
    // its items staging -> tile buffer (decode).
    int bt_next = 0;  // wave 0: block-table entry of key `lane` of the tile put next
    auto issue_bt = [&](int t) {
        const int pos = t * kKT + lane;
        if (wave == 0 && pos < kv_end) {
            const int lb = a.bs_shift >= 0 ? pos >> a.bs_shift : pos / a.block_size;
            bt_next = a.bt[seq * a.bt_ss + lb];
        }
    };
    auto put_offsets = [&](int t) {
        if (wave == 0) {
            const int pos = t * kKT + lane;
            uint64_t off = 0;  // keys past the visible range read slot 0 (their norms are zeroed)
            if (pos < kv_end) {
                const int o = a.bs_shift >= 0 ? pos & (a.block_size - 1) : pos % a.block_size;
                const int64_t phys = (bt_next < 0 || bt_next >= a.num_blocks) ? 0 : bt_next;
                off = (uint64_t)(phys * a.stride_block + (int64_t)o * a.stride_token);
            }
            soff[lane] = off;
        }
    };
    auto stage = [&]() {
        for (int c = wave; c < kCopies; c += nwaves) {
            int key, byte_off, dst;
            bool on = true;
            if (c < 32) {  // index dwords: keys 4 (c % 16) + lane / 16, dword lane % 16
                const bool isk = c < 16;
                key = 4 * (c & 15) + (lane >> 4);
                byte_off = (isk ? SL.k_idx : SL.v_idx) + h * SL.ib + 4 * (lane & 15);
                dst = (isk ? kSKi : kSVi) + (c & 15) * 256;
                on = 4 * (lane & 15) < SL.ib;  // the dense layout has 12 index dwords per head
            } else {  // norms: key = lane
                key = lane;
                byte_off = (c == 32 ? SL.k_norm : SL.v_norm) + 4 * h;
                dst = c == 32 ? kSKn : kSVn;
            }
            const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds0 + dst);
            if (on) copy4(a.cache + soff[key] + byte_off, m0);
        }
    };
    // Returns the tile's V exponent e: 2^e above its largest v norm, clamped to
    // [-14, 24] so that 2^-e is an fp16 value (the row-sum MFMA reads it).
    auto decode = [&](int t) -> int {
        uint8_t *tb = lds + (t & 1) * kTileBytes;
        const int nk = min(kKT, kv_end - t * kKT);  // keys past it get norm 0
        const float *kn = reinterpret_cast<const float *>(lds + kSKn);
        const float *vn = reinterpret_cast<const float *>(lds + kSVn);
        float vx = lane < nk ? fmaxf(vn[lane], 0.f) : 0.f;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) vx = fmaxf(vx, __shfl_xor(vx, o));
        const int e_v = min(24, max(-14, (int)((__float_as_uint(vx) >> 23) & 0xffu) - 126));
        const float vs = ldexpf(1.f, -e_v);
        for (int w = tid; w < kItems; w += nthr) {
            if (w < 256) {
                // K rows: key r, dims 32 qq .. 32 qq + 31 (index dwords 4 qq .. 4 qq + 3).  The
                // key's 16-bit table dtype(centroid * norm) of every codebook entry is built in
                // registers, and its 32 indices are looked up with byte permutes; a piece holds
                // dims 8c .. 8c+7 in the order e0 e2 e4 e6 e1 e3 e5 e7 (the query operand's).
                const int r = w >> 2, qq = w & 3;
                const float nrm = r < nk ? kn[r] : 0.f;
                Table16 tab;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    uint32_t pr[2];
#pragma unroll
                    for (int h2 = 0; h2 < 2; ++h2) {
                        const int j = 4 * c + 2 * h2;
                        pr[h2] = Elem<DT>::from_f32(opaque(ktab[j] * nrm)) |
                                 (Elem<DT>::from_f32(opaque(ktab[j + 1] * nrm)) << 16);
                    }
                    tab.lo[c] = perm(pr[1], pr[0], 0x06040200u);  // low bytes of entries 4c .. 4c+3
                    tab.hi[c] = perm(pr[1], pr[0], 0x07050301u);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int dw = 4 * qq + i;
                    const uint32_t x = idx_dword(lds + kSKi + r * 64, dw, a.dense3 != 0);
                    const uint32_t ev = (x >> 4) & 0x0f0f0f0fu, od = x & 0x0f0f0f0fu;
                    uint2 e, o;
                    if (a.nkc <= 8) {
                        e = lookup4<3>(tab, ev);
                        o = lookup4<3>(tab, od);
                    } else {
                        e = lookup4<4>(tab, ev);
                        o = lookup4<4>(tab, od);
                    }
                    *reinterpret_cast<u32x4 *>(tb + kTK + kt_piece(r, dw)) = u32x4{e.x, e.y, o.x, o.y};
                }
            } else {  // V'^T rows 8 dw + 2j + par, keys 4 tq .. 4 tq + 3 (8 bytes each)
                const int u = w - 256;
                const int tq = u & 15, dw = u >> 4;
                const int t0 = 4 * tq;
                const int b = t0 >> 4, gg = (t0 >> 2) & 3;
                const int piece = 4 * (b >> 1) + gg, elem_off = 8 * (b & 1);
                uint32_t x[4];
                float nrm[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[i] = idx_dword(lds + kSVi + (t0 + i) * 64, dw, a.dense3 != 0);
                    nrm[i] = t0 + i < nk ? vn[t0 + i] : 0.f;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int par = 0; par < 2; ++par) {
                        const int d = 8 * dw + 2 * j + par;
                        uint32_t e[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint32_t idx = (x[i] >> (8 * j + (par ? 0 : 4))) & 15u;
                            // V in the q dtype, then scaled into fp16 (exact in fp16 range)
                            const float v = Elem<DT>::to_f32(Elem<DT>::from_f32(opaque(vtab[idx] * nrm[i])));
                            e[i] = f32_to_f16_bits(v * vs);
                        }
                        *reinterpret_cast<uint2 *>(tb + kTVt + vt_piece(d, piece) + elem_off) =
                            make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
                    }
                }
            }
        }
        return e_v;
    };

    // prologue: offsets of tile 0, its copies in flight while the query operand is built
    if (n_tiles > 0) {
        issue_bt(0);
        put_offsets(0);
    }
    __syncthreads();  // offsets of tile 0, codebook tables
    if (n_tiles > 0) stage();
    if (n_tiles > 1) issue_bt(1);

    // ---- Q^T operand: position i0 + col, k-step s = dims 32s + 8g .. +7 of q_rot ----
    u32x4 qop[4];
    {
        const int qi = i0 + col;
        const bool qvalid = wave_active && qi < T;
        const uint16_t *qrow = reinterpret_cast<const uint16_t *>(a.q) + (int64_t)(q0 + (qvalid ? qi : 0)) * a.q_st +
                               (int64_t)hq * a.q_sh;
#pragma unroll
        for (int s_ = 0; s_ < 4; ++s_) {
            const int base = 32 * s_ + 8 * g;
            const uint4 rw = qvalid ? *reinterpret_cast<const uint4 *>(qrow + base) : make_uint4(0, 0, 0, 0);
            const uint32_t w16[4] = {rw.x, rw.y, rw.z, rw.w};
            float xin[8], qr[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) xin[k] = Elem<DT>::to_f32((w16[k >> 1] >> (16 * (k & 1))) & 0xffffu);
            rotate_q8<DT>(xin, base, a.R, a.rot_block, qr);
            // dims in the K rows' order e0 e2 e4 e6 e1 e3 e5 e7
            uint32_t pk[4];
            constexpr int ord[8] = {0, 2, 4, 6, 1, 3, 5, 7};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                pk[k] = Elem<DT>::from_f32(qr[ord[2 * k]]) | (Elem<DT>::from_f32(qr[ord[2 * k + 1]]) << 16);
            qop[s_] = u32x4{pk[0], pk[1], pk[2], pk[3]};
        }
    }

    int e_cur = 0;
    if (n_tiles > 0) {
        wait_copies<0>();
        __syncthreads();  // tile 0 staged
        e_cur = decode(0);
        if (n_tiles > 1) put_offsets(1);
        __syncthreads();  // tile 0 decoded, offsets of tile 1
    }

    AttnState st;
    st.init();
    for (int ti = 0; ti < n_tiles; ++ti) {
        const int k0 = ti * kKT;
        const int nk = min(kKT, kv_end - k0);
        const bool more = ti + 1 < n_tiles;
        if (more) stage();                        // tile ti + 1 -> staging
        if (ti + 2 < n_tiles) issue_bt(ti + 2);  // its block-table entries, read after the compute
        const uint8_t *tb = lds + (ti & 1) * kTileBytes;
        // (every wave reaches the barriers below)
        if (wave_active && (!a.causal || k0 <= pos_base + i0 + kPQ - 1)) {
            // ---- S^T = K Q^T for 4 key blocks of 16 ----
            float s[16];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                f32x4 c = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    // key 16b + col, piece 4ks + g (the swizzle term of key 16b + col is col)
                    const u32x4 kv = *reinterpret_cast<const u32x4 *>(tb + kTK + kt_piece(16 * b + col, 4 * ks + g));
                    c = mfma_qk<DT>(kv, qop[ks], c);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) s[4 * b + i] = c[i];
            }
            // causal and tile-end mask: key < min(k0 + nk, position + 1)
            const bool full = nk == kKT && (!a.causal || k0 + kKT - 1 <= pos_base + i0);
            if (!full) {
                const int lim = (a.causal ? min(k0 + nk, my_pos + 1) : k0 + nk) - (k0 + 4 * g);
#pragma unroll
                for (int j = 0; j < 16; ++j) s[j] = (16 * (j >> 2) + (j & 3)) < lim ? s[j] : -INFINITY;
            }
            softmax_pv(st, s, a.score_scale, 1.f, e_cur, tb + kTVt, voff0, voff1, rowsum_operand(e_cur, col));
        }
        if (more) {
            wait_copies<0>();
            __syncthreads();  // tile ti + 1 staged (and every wave done with the offsets)
            e_cur = decode(ti + 1);
            if (ti + 2 < n_tiles) put_offsets(ti + 2);
            __syncthreads();  // tile ti + 1 decoded; staging and offsets free again
        }
    }
    if (!wave_active) return;

    const float inv_l = attn_inv_l(st);
    if (i0 + col >= T) return;
    uint16_t *orow = reinterpret_cast<uint16_t *>(a.out) + (int64_t)(q0 + i0 + col) * a.o_st + (int64_t)hq * a.o_sh;
    store_rotated<DT>(st, inv_l, orow, a.R, a.rot_block, g);
}

}  // namespace

}  // namespace rq

using namespace rq;

extern "C" int rq_paged_attention(const void *q, int32_t dtype, int64_t total_q, int32_t num_q_heads,
                                  int64_t q_stride_tok, int64_t q_stride_head, const int32_t *cu_seqlens_q,
                                  int64_t num_seqs, int64_t max_q_len, int32_t causal, const uint8_t *kv_cache,
                                  int64_t num_blocks, int32_t block_size, int64_t stride_block, int64_t stride_token,
                                  int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                                  const int32_t *block_table,
                                  int64_t max_blocks, int64_t bt_stride_seq, const int32_t *seq_lens,
                                  const float *k_centroids, int32_t n_k_centroids, const float *v_centroids,
                                  int32_t n_v_centroids, const float *rotation, int32_t rot_block, float sm_scale,
                                  void *out, int64_t out_stride_tok, int64_t out_stride_head, void *stream) {
    RQ_CHECK_ARG(dtype == RQ_DTYPE_BF16 || dtype == RQ_DTYPE_F16, "attention dtype must be f16 or bf16");
    RQ_CHECK_ARG(head_dim == kD, "head_dim %d unsupported (only %d)", head_dim, kD);
    RQ_CHECK_ARG(num_kv_heads >= 1 && num_q_heads % num_kv_heads == 0 && num_q_heads / num_kv_heads <= 16,
                 "num_q_heads %d / num_kv_heads %d must be an integer <= 16", num_q_heads, num_kv_heads);
    RQ_CHECK_ARG(n_k_centroids >= 1 && n_k_centroids <= 16 && n_v_centroids >= 1 && n_v_centroids <= 16,
                 "centroid counts must be 1..16");
    RQ_CHECK_ARG(rot_block == 2 || rot_block == 4, "rot_block %d must be 2 or 4", rot_block);
    RQ_CHECK_ARG(num_seqs >= 0 && total_q >= 0 && max_q_len >= 0 && block_size >= 1 && max_blocks >= 0 &&
                     num_blocks >= 0,
                 "bad sizes");
    const int lrc = check_index_layout(index_layout, head_dim, n_k_centroids, n_v_centroids);
    if (lrc) return lrc;
    RQ_CHECK_ARG(stride_token % 4 == 0 && stride_block % 4 == 0 && ((uintptr_t)kv_cache % 4) == 0,
                 "cache slots must be 4-byte aligned");
    RQ_CHECK_ARG(((uintptr_t)q % 16) == 0 && (q_stride_tok * 2) % 16 == 0 && (q_stride_head * 2) % 16 == 0,
                 "q rows must be 16-byte aligned");
    RQ_CHECK_ARG(((uintptr_t)out % 8) == 0 && (out_stride_tok * 2) % 8 == 0 && (out_stride_head * 2) % 8 == 0,
                 "out rows must be 8-byte aligned");
    RQ_CHECK_ARG(((uintptr_t)rotation % 16) == 0, "rotation must be 16-byte aligned");
    if (num_seqs == 0 || max_q_len == 0 || total_q == 0) return RQ_OK;
    RQ_CHECK_ARG(num_blocks >= 1, "the cache has no blocks");
    AttnArgs a{};
    a.q = q;
    a.q_st = q_stride_tok;
    a.q_sh = q_stride_head;
    a.cu_q = cu_seqlens_q;
    a.cache = kv_cache;
    a.stride_block = stride_block;
    a.stride_token = stride_token;
    a.block_size = block_size;
    a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
    a.num_blocks = num_blocks;
    a.H = num_kv_heads;
    a.G = num_q_heads / num_kv_heads;
    a.dense3 = index_layout == RQ_INDEX_DENSE3;
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
    a.causal = causal != 0;
    a.score_scale = sm_scale * kAttnLog2e;
    // GQA groups of more than kMaxWaves heads go to hsplit workgroups per kv head
    // (the smallest split into equal parts of at most kMaxWaves heads); then
    // 16-position groups per workgroup: up to kMaxWaves waves for long queries,
    // at least kMinWaves waves (they share the tile decode).  When every query is
    // short (one position group), the workgroup has kMaxWaves waves anyway: the
    // waves past the GQA group's only decode tiles, which is most of a
    // decode-shaped call's time.
    a.hsplit = 1;
    while (a.G % a.hsplit != 0 || a.G / a.hsplit > kMaxWaves) ++a.hsplit;
    const int gw = a.G / a.hsplit;
    a.npg = max_q_len > kPQ ? std::max(1, kMaxWaves / gw) : 1;
    if (max_q_len > kPQ)
        while (gw * a.npg < kMinWaves) ++a.npg;
    a.qb = kPQ * a.npg;
    a.ncomp = gw * a.npg;
    a.out = out;
    a.o_st = out_stride_tok;
    a.o_sh = out_stride_head;
    const int nwaves = max_q_len > kPQ ? a.ncomp : kMaxWaves;
    dim3 grid((unsigned)((max_q_len + a.qb - 1) / a.qb), (unsigned)(a.H * a.hsplit), (unsigned)num_seqs);
    const size_t lds = kLdsBytes;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == RQ_DTYPE_BF16)
        hipLaunchKernelGGL((paged_attn_kernel<RQ_DTYPE_BF16>), grid, dim3(64 * nwaves), lds, st, a);
    else
        hipLaunchKernelGGL((paged_attn_kernel<RQ_DTYPE_F16>), grid, dim3(64 * nwaves), lds, st, a);
    return check_launch("paged_attn_kernel");
}
