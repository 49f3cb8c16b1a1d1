// Causal prefill attention over the packed RotorQuant cache on int8 MFMA (gfx950).
//
// Replaces fused_paged_rq_int8_prefill
// (src/rotorquant_vllm/triton/fused_paged_rq_int8_prefill.py:247-363, kernel :43-239):
// attention in the rotated space, q_rot = q R^T rounded to the q dtype, output
// rounded and rotated back by R.  Differences from the reference, on purpose:
//   * any number of sequences per launch (cu_seqlens_q), and query i of a
//     sequence sits at position seq_len - q_len + i (chunked prefill with a
//     cached prefix is causal-correct; the reference places it at i);
//   * key tiles entirely above the causal diagonal are skipped;
//   * int8 operands are rounded to nearest and carry a second int8 "low" part,
//     one int8 being too coarse for the 2e-2 output tolerance:
//       Q K^T = s_q s_k [q_hi.k_hi + (q_hi.k_lo + q_lo.k_hi) / 128]   (3 int8 MFMAs)
//     q per query row (absmax / 127); k per 64-key tile: the reference's K,
//     centroid * norm rounded to the q dtype (:172), in units of s_tile / 127,
//     s_tile = dtype(max|centroid| * largest k norm of the tile) >= every |k|.
//   P V runs on the fp16 MFMA, as the reference's 16-bit product (:217-227) but
//   with 11-bit operands on both sides: V' = V * 2^-e_tile in fp16, V the
//   reference's centroid * norm rounded to the q dtype (:224), 2^e_tile above the
//   64-key tile's largest v norm, and P' = p * 2^(e_tile - e_run) in fp16, e_run
//   the largest e_tile so far (acc is rescaled when it grows); the row sum is a
//   17th MFMA row of 2^-e_tile.
//
// Two kernels per call:
//   * prefill_pack_kernel decodes every 64-key tile of every (sequence, kv head)
//     once into a "tile image" in the caller's workspace: K hi/lo int8 rows (key
//     norms included), fp16 V'^T rows, the tile's score unit and V exponent,
//     laid out exactly as the attention kernel keeps them in LDS;
//   * prefill_attn_kernel: one workgroup per (query block of QB positions, kv
//     head, sequence); its waves are (query head of the GQA group, 16-position
//     group).  It streams the tile images of its sequence and kv head into a
//     double-buffered LDS area with direct global -> LDS copies (the copy of
//     tile t+1 runs while tile t is computed), so the inner loop is MFMA,
//     softmax and the int8 quantization of P only.
// MFMA v_mfma_i32_16x16x64_i8 (wave64, lane l, g = l / 16):
//   A (16 x 64): lane holds row l % 16, k = 16g .. 16g+15 (16 bytes)
//   B (64 x 16): lane holds col l % 16, k = 16g .. 16g+15
//   C (16 x 16): lane holds col l % 16, rows 4g .. 4g+3 (4 int32)
// S^T = K Q^T: rows = 16 keys of a key block, cols = 16 query positions; lane
// (g, col) then holds the scores of keys 16b + 4g + i (b, i = 0..3).
// O^T = V^T P^T on v_mfma_f32_16x16x32_f16 (A 16 x 32: lane holds row
// l % 16, k = 8g .. 8g+7), two k-steps per tile: k-step s, element j of lane
// group g is key 32s + 4g + j (j < 4) or 32s + 16 + 4g + j - 4 (j >= 4) --
// exactly the scores the lane holds, so P needs no transpose.
#include <algorithm>

#include "rq_attn_tile.h"

namespace rq {

constexpr int kPD = kAttnD;   // head_dim
constexpr int kKT = kAttnKT;  // keys per tile
constexpr int kPQ = kAttnPQ;  // query positions per wave
constexpr float kLog2eP = kAttnLog2e;

__device__ __forceinline__ i32x4 mfma_i8(u32x4 a, u32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0,
                                                 0);
}


__device__ __forceinline__ int sat_i8(float x) { return (int)fminf(127.f, fmaxf(-127.f, rintf(x))); }

struct PrefillArgs {
    const void *q;
    int64_t q_st, q_sh;
    const int32_t *cu_q;
    const uint8_t *cache;
    int64_t stride_block, stride_token;
    int block_size, bs_shift;
    int64_t num_blocks;
    int H, G, HQ;
    int dense3;         // dense 3-bit index layout of the cache
    const int32_t *bt;
    int64_t bt_ss, max_blocks;
    const int32_t *seq_lens;
    const float *kc, *vc;
    int nkc, nvc;
    const float *R;
    int rot_block;
    float score_scale;  // sm_scale * log2(e)
    int causal;         // 0: every query sees all seq_lens[b] keys
    int qb;             // query positions per workgroup (= 16 * position groups)
    int npg;            // position groups per workgroup
    int flat;           // 1: workgroups of 8 waves over the sequence's (position group, query head) units
    int64_t max_tiles;  // tile images per (sequence, kv head) in the workspace
    uint8_t *ws;        // tile images [num_seqs][H][max_tiles][kImBytes]
    void *out;
    int64_t o_st, o_sh;
};

// Tile image (bytes), the same in the workspace and in LDS.  Rows are unpadded;
// their 16-byte pieces are stored XOR-swizzled so that the ds_read_b128 operand
// reads of an MFMA (16 lanes: 16 rows, one piece each) run without bank
// conflicts.  Padded pitches of 144 / 80 bytes measured two-way conflicts on
// gfx950; these swizzles measured conflict-free (same speed as contiguous reads).
//   K row r, piece c (0..7):   r * 128 + 16 * (c ^ (r & 7))
//   V^T row d, piece c (0..7): the same (8 keys of 16 bits per piece)
// K operand modes of the tile image and the attention kernel:
//   kKqInt8: K hi/lo int8 rows (the int8 prefill, rq_int8_prefill);
//   kKqDtype: K rows in the q dtype, dtype(centroid * norm) -- the reference's
//     non-fused numerics (K and V rounded to the q dtype, rq_paged_prefill) --
//     as two [64 keys][64 dims] halves in the same 16 KB and the same swizzle
//     (piece c of key r's half h holds dims 64h + 8c .. +7 in order).
constexpr int kKqInt8 = 0, kKqDtype = 1;
constexpr int kKP = kPD;                            // K row pitch
constexpr int kImKhi = 0;                           // [64 keys][kKP] int8, dims permuted per 8
constexpr int kImKlo = kImKhi + kKT * kKP;          // same, low parts
constexpr int kImVt = kImKlo + kKT * kKP;          // [128 dims][64 keys] fp16 V', keys in MFMA k order
__host__ __device__ constexpr int k_piece(int r, int c) { return r * kKP + 16 * (c ^ (r & 7)); }
// V^T row d (128 bytes: 8 pieces of 8 keys) uses the K row swizzle: piece c at k_piece(d, c).
constexpr int kImSk = kImVt + kPD * kKT * 2;        // float: score unit = s_tile / 127 * score_scale / 128 (int8 K)
constexpr int kImVe = kImSk + 4;                    // int: e_tile, 2^e_tile > the tile's largest v norm
constexpr int kImOnes = kImSk + 16;                 // row-sum operand: 4 dwords of 2^-e_tile (fp16 pair), 4 zero dwords
constexpr int kImBytes = (kImOnes + 32 + 1023) / 1024 * 1024;  // whole 1 KB copies
constexpr int kImChunks = kImBytes / 1024;

// Largest |centroid| of a codebook (1 when all are zero): int8 unit = this / 127.
__device__ __forceinline__ float codebook_max(const float *c, int n) {
    float m = 0.f;
    for (int e = 0; e < n; ++e) m = fmaxf(m, fabsf(c[e]));
    return m > 0.f ? m : 1.f;
}

// Keys of a sequence the attention may read: its length, bounded by the block
// table's capacity and by the workspace's tile images.
__device__ __forceinline__ int visible_keys(const PrefillArgs &a, int64_t seq) {
    const int64_t cap = min(a.max_blocks * a.block_size, a.max_tiles * kKT);
    return (int)min((int64_t)a.seq_lens[seq], cap);
}

// ---- pack: one workgroup (256 threads) per (tile, kv head, sequence) --------
template <int DT, int KQ>
__global__ __launch_bounds__(256) void prefill_pack_kernel(PrefillArgs a) {
    const int tile = blockIdx.x, h = blockIdx.y;
    const int64_t seq = blockIdx.z;
    const int L_eff = visible_keys(a, seq);
    const int k0 = tile * kKT;
    if (k0 >= L_eff) return;
    const int nk = min(kKT, L_eff - k0);
    const int tid = threadIdx.x;
    uint8_t *img = a.ws + (((int64_t)seq * a.H + h) * a.max_tiles + tile) * kImBytes;
    const SlotLayout SL(a.H, kPD, a.dense3 != 0);
    __shared__ uint64_t toff[kKT];
    const float kmax = codebook_max(a.kc, a.nkc);

    // K and V are the reference's values, dtype(centroid * norm), in both modes.  int8
    // K: in units of s_tile / 127 (s_tile = dtype(kmax * largest k norm of the tile),
    // the largest |k| the tile can hold, as rounding is monotone), so the key norms
    // are part of the K operand and the score unit is one per tile.
    __shared__ float ktab[16], vtab[16];
    __shared__ float knorm[kKT], vnorm[kKT];
    __shared__ float vscale;  // 2^-e_v
    __shared__ float kinv;    // 127 / s_tile (int8 K)
    if (tid < 16) {
        ktab[tid] = tid < a.nkc ? a.kc[tid] : 0.f;
        vtab[tid] = tid < a.nvc ? a.vc[tid] : 0.f;
    }
    if (tid < kKT) {
        // token offset (keys past the tile's end read slot 0 and get zero norms)
        uint64_t off = 0;
        float nkv = 0.f, nvv = 0.f;
        if (tid < nk) {
            const int pos = k0 + tid;
            int lb, o;
            if (a.bs_shift >= 0) {
                lb = pos >> a.bs_shift;
                o = pos & (a.block_size - 1);
            } else {
                lb = pos / a.block_size;
                o = pos - lb * a.block_size;
            }
            int64_t phys = a.bt[seq * a.bt_ss + lb];
            phys = (phys < 0 || phys >= a.num_blocks) ? 0 : phys;
            off = (uint64_t)(phys * a.stride_block + (int64_t)o * a.stride_token);
            nkv = *reinterpret_cast<const float *>(a.cache + off + SL.k_norm + 4 * h);
            nvv = *reinterpret_cast<const float *>(a.cache + off + SL.v_norm + 4 * h);
        }
        toff[tid] = off;
        // tile scales: the largest k norm; the power of two above the largest v norm
        float kx = fmaxf(nkv, 0.f), vx = fmaxf(nvv, 0.f);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            kx = fmaxf(kx, __shfl_xor(kx, o));
            vx = fmaxf(vx, __shfl_xor(vx, o));
        }
        const float s_raw = Elem<DT>::to_f32(Elem<DT>::from_f32(opaque(kmax * kx)));
        const float s_tile = s_raw > 0.f ? s_raw : 1.f;
        // 2^e_v > vx, clamped to [-14, 24] so that 2^-e_v is an fp16 (normal or denormal)
        // value: the attention kernel's row-sum MFMA reads it.  Norms above 2^24 would
        // overflow v' in fp16.
        const int e_v = min(24, max(-14, (int)((__float_as_uint(vx) >> 23) & 0xffu) - 126));
        knorm[tid] = nkv;
        vnorm[tid] = nvv;
        if (tid == 0) {
            *reinterpret_cast<float *>(img + kImSk) =
                KQ == kKqInt8 ? s_tile * (1.f / 127.f) * a.score_scale * (1.f / 128.f) : a.score_scale;
            kinv = 127.f / s_tile;
            *reinterpret_cast<int *>(img + kImVe) = e_v;
            const uint32_t w = pack_f16(ldexpf(1.f, -e_v), ldexpf(1.f, -e_v));
            *reinterpret_cast<u32x4 *>(img + kImOnes) = u32x4{w, w, w, w};
            *reinterpret_cast<u32x4 *>(img + kImOnes + 16) = u32x4{0u, 0u, 0u, 0u};
            vscale = ldexpf(1.f, -e_v);
        }
    }
    __syncthreads();
    // This thread's index dwords -- K: (key, dword) w = tid + 256 r, r < 4; V: dword
    // tid >> 4 of the keys of quad tid & 15 -- all loaded before the first image store:
    // a load issued after a store would wait for it (the compiler cannot rule out that
    // they alias, and the memory counter completes in order), one round per loop step.
    static_assert(kKT * 16 == 4 * 256, "four K index dwords per thread");
    uint32_t xk[4], xv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int w = tid + 256 * r;
        xk[r] = idx_dword(a.cache + toff[w >> 4] + SL.k_idx + h * SL.ib, w & 15, a.dense3 != 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
        xv[i] = idx_dword(a.cache + toff[4 * (tid & 15) + i] + SL.v_idx + h * SL.ib, tid >> 4, a.dense3 != 0);
    if constexpr (KQ == kKqDtype) {
        // K rows in the q dtype: dims 8 dw .. 8 dw + 7 of key tk, one 16-byte piece
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int w = tid + 256 * r;
            const int tk = w >> 4, dw = w & 15;
            const uint32_t x = xk[r];
            const float nrm = knorm[tk];
            uint32_t pr[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {  // byte j: dim 8 dw + 2j in the high nibble, + 1 in the low one
                const uint32_t e0 = Elem<DT>::from_f32(opaque(ktab[(x >> (8 * j + 4)) & 15u] * nrm));
                const uint32_t e1 = Elem<DT>::from_f32(opaque(ktab[(x >> (8 * j)) & 15u] * nrm));
                pr[j] = e0 | (e1 << 16);
            }
            *reinterpret_cast<u32x4 *>(img + kImKhi + (dw >> 3) * (kKT * kKP) + k_piece(tk, dw & 7)) =
                u32x4{pr[0], pr[1], pr[2], pr[3]};
        }
    } else
    // K rows (dims permuted per 8 as e0 e2 e4 e6 e1 e3 e5 e7), hi and lo
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int w = tid + 256 * r;
        const int tk = w >> 4, dw = w & 15;  // token, dword of the head's 64 index bytes
        const uint32_t x = xk[r];
        const float nrm = knorm[tk], inv = kinv;
        uint32_t hw[2], lw[2];  // [0]: even dims (high nibbles), [1]: odd dims (low nibbles)
#pragma unroll
        for (int par = 0; par < 2; ++par) {
            uint32_t hv = 0, lv = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // the reference's K, dtype(c * n) (|k| <= s_tile), in units of s_tile / 127
                const float kr = Elem<DT>::to_f32(Elem<DT>::from_f32(opaque(ktab[(x >> (8 * j + (par ? 0 : 4))) & 15u] * nrm)));
                const float t = kr * inv;  // |t| <= 127
                const int hi = sat_i8(t);
                const int lo = sat_i8((t - (float)hi) * 128.f);
                hv |= (uint32_t)(hi & 0xff) << (8 * j);
                lv |= (uint32_t)(lo & 0xff) << (8 * j);
            }
            hw[par] = hv;
            lw[par] = lv;
        }
        const int ko = k_piece(tk, dw >> 1) + 8 * (dw & 1);
        *reinterpret_cast<uint2 *>(img + kImKhi + ko) = make_uint2(hw[0], hw[1]);
        *reinterpret_cast<uint2 *>(img + kImKlo + ko) = make_uint2(lw[0], lw[1]);
    }
    // V'^T rows: v' = dtype(centroid * norm) * 2^-e_v (exact), rounded to fp16 (exact
    // unless below fp16's normal range; |v'| < max|centroid|).  Key t = 16b + 4gg + i sits in piece
    // 4 (b >> 1) + gg of its dim row, element 4 (b & 1) + i: thread (key quad,
    // dword) writes 4 consecutive keys = 8 bytes.
    {
        const int tq = tid & 15, dw = tid >> 4;  // key quad (4 consecutive keys), dword position
        const uint32_t(&x)[4] = xv;
        const int t0 = 4 * tq;
        const int b = t0 >> 4, gg = (t0 >> 2) & 3;
        const int piece = 4 * (b >> 1) + gg, elem_off = 8 * (b & 1);
        float nv[4];
        const float vs = vscale;
#pragma unroll
        for (int i = 0; i < 4; ++i) nv[i] = vnorm[t0 + i];
#pragma unroll
        for (int j = 0; j < 4; ++j) {  // byte j of the dword: dims 8 dw + 2j (high nibble), + 1 (low)
#pragma unroll
            for (int par = 0; par < 2; ++par) {
                const int d = 8 * dw + 2 * j + par;
                uint32_t e[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t idx = (x[i] >> (8 * j + (par ? 0 : 4))) & 15u;
                    // V rounded to the q dtype first, as the reference (fused_paged_rq_int8_prefill.py:224)
                    const float v = Elem<DT>::to_f32(Elem<DT>::from_f32(opaque(vtab[idx] * nv[i])));
                    e[i] = f32_to_f16_bits(v * vs);
                }
                *reinterpret_cast<uint2 *>(img + kImVt + k_piece(d, piece) + elem_off) =
                    make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
            }
        }
    }
}

template <int DT, int KQ>
__global__ __launch_bounds__(1024) void prefill_attn_kernel(PrefillArgs a) {
    int qblk, h;
    int64_t seq;
    attn_work_item(qblk, h, seq);
    const int q0 = a.cu_q[seq], q1 = a.cu_q[seq + 1];
    const int T = q1 - q0;
    const int L = a.seq_lens[seq];
    const int pos_base = L - T;  // position of query 0
    const int L_eff = visible_keys(a, seq);
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int nwaves = nthr >> 6;
    // This wave's query head inside the GQA group (gh) and first query index (i0), and
    // the workgroup's last query index.  Plain: wave = (gh, position group pg) of the
    // workgroup's npg groups.  Flat (GQA groups whose G * npg waves would not spread
    // evenly over a CU's four SIMDs, e.g. 7): the sequence's (position group, query
    // head) units in position-group-major order, nwaves consecutive units per
    // workgroup (at most two position groups when G < 8).
    int gh, i0, last_i;
    if (a.flat) {
        const int units = T > 0 ? (T + kPQ - 1) / kPQ * a.G : 0;
        const int f0 = qblk * nwaves;
        if (f0 >= units) return;
        const int f = f0 + wave;
        gh = f % a.G;
        i0 = f < units ? f / a.G * kPQ : T;  // units past the end: inactive
        last_i = min(T, (min(f0 + nwaves, units) - 1) / a.G * kPQ + kPQ) - 1;
    } else {
        if (qblk * a.qb >= T || T <= 0) return;
        gh = wave / a.npg;
        const int pg = wave - gh * a.npg;  // 16-position group
        i0 = qblk * a.qb + pg * kPQ;
        last_i = min(T, (qblk + 1) * a.qb) - 1;
    }
    const int g = lane >> 4, col = lane & 15;
    // this lane's operand pieces in a tile image: key col, pieces g and 4 + g; dim col, piece g
    const int koff0 = k_piece(col, g), koff1 = k_piece(col, 4 + g);
    const int ones_off = kImOnes + (col == 0 ? 0 : 16);  // the row-sum operand (MFMA row 0 = col 0)
    const int hq = h * a.G + gh;
    const bool wave_active = i0 < T;
    const int my_i = i0 + col;              // query index of this lane's column
    const int my_pos = pos_base + my_i;

    // LDS: two tile-image buffers.
    extern __shared__ __align__(16) uint8_t lds[];

    // ---- key range: causal bound of the whole workgroup --------------------------
    const bool causal = KQ == kKqInt8 || a.causal;  // the int8 prefill is always causal
    const int kv_end = causal ? min(L_eff, pos_base + last_i + 1) : L_eff;  // keys [0, kv_end) may be visible
    const int n_tiles = (kv_end + kKT - 1) / kKT;

    // Tile images of this (sequence, kv head), copied global -> LDS 1 KB per wave
    // instruction into two buffers; tile t+1's copy runs while tile t is computed.
    // Tiles 0 and 1 are issued first, so that their copies overlap the query
    // operand's loads and arithmetic (the query operand uses no LDS).
    const uint8_t *img0 = a.ws + ((int64_t)seq * a.H + h) * a.max_tiles * kImBytes;
    const uint32_t lds0 = lds_addr(lds);
    auto issue_tile = [&](int t) {
        const uint8_t *src = img0 + (int64_t)t * kImBytes;
        const uint32_t dst = lds0 + (t & 1) * kImBytes;
        for (int c = wave; c < kImChunks; c += nwaves) {
            // wave-uniform operands of the copy (the compiler cannot prove it here)
            const uint64_t s = reinterpret_cast<uint64_t>(src + c * 1024);
            const uint32_t slo = __builtin_amdgcn_readfirstlane((uint32_t)s);
            const uint32_t shi = __builtin_amdgcn_readfirstlane((uint32_t)(s >> 32));
            const uint8_t *su = reinterpret_cast<const uint8_t *>(((uint64_t)shi << 32) | slo);
            copy16(su, 16 * lane, __builtin_amdgcn_readfirstlane(dst + c * 1024));
        }
    };
    if (n_tiles > 0) issue_tile(0);
    if (n_tiles > 1) issue_tile(1);

    // ---- Q^T operand (cols = this wave's 16 positions): q_rot rounded to the q dtype,
    //      quantised per position to hi/lo int8, dims in the permuted order of K ----
    u32x4 qh[2], ql[2];
    float sq = KQ == kKqInt8 ? 0.f : 1.f;
    if (KQ == kKqDtype && wave_active) {
        // q-dtype K: the operand is q_rot rounded to the q dtype, k-step s = dims 32s + 8g .. +7
        const int qi = i0 + col;
        const bool qvalid = qi < T;
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
            uint32_t pk[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) pk[k] = Elem<DT>::from_f32(qr[2 * k]) | (Elem<DT>::from_f32(qr[2 * k + 1]) << 16);
            (s_ < 2 ? qh[s_] : ql[s_ - 2]) = u32x4{pk[0], pk[1], pk[2], pk[3]};
        }
    }
    if (KQ == kKqInt8 && wave_active) {
        // Lane (g, col) holds the operand of position i0 + col at dims 64s + 16g .. +15
        // (s = 0, 1): it rotates exactly those 32 dims (rotation blocks are aligned
        // to 2 or 4 dims), q_rot rounded to the q dtype.
        const int qi = i0 + col;
        const bool qvalid = qi < T;
        const uint16_t *qrow = reinterpret_cast<const uint16_t *>(a.q) + (int64_t)(q0 + (qvalid ? qi : 0)) * a.q_st +
                               (int64_t)hq * a.q_sh;
        const int rb = a.rot_block;
        float qr[32];  // [s][16]: dims 64s + 16g + k
#pragma unroll
        for (int s_ = 0; s_ < 2; ++s_) {
            const int base = 64 * s_ + 16 * g;
            uint4 raw[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
            if (qvalid) {
                raw[0] = *reinterpret_cast<const uint4 *>(qrow + base);
                raw[1] = *reinterpret_cast<const uint4 *>(qrow + base + 8);
            }
            const uint32_t w16[8] = {raw[0].x, raw[0].y, raw[0].z, raw[0].w, raw[1].x, raw[1].y, raw[1].z, raw[1].w};
            float xin[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) xin[k] = Elem<DT>::to_f32((w16[k >> 1] >> (16 * (k & 1))) & 0xffffu);
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) rotate_q8<DT>(xin + 8 * hf, base + 8 * hf, a.R, rb, qr + 16 * s_ + 8 * hf);
        }
        // per-position absmax over 128 dims: this lane's 32, then the other three lane groups
        float amax = 0.f;
#pragma unroll
        for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(qr[k]));
        amax = rows_max(amax);
        sq = amax > 0.f ? amax / 127.f : 1.f;
        const float inv = 1.f / sq;
        // k-step s covers dims 64s .. 64s+63; lane group g holds dims 64s + 16g .. +15,
        // stored as two 8-dim groups in the order e0 e2 e4 e6 e1 e3 e5 e7.
#pragma unroll
        for (int s_ = 0; s_ < 2; ++s_) {
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
                uint32_t h2[2] = {0, 0}, l2[2] = {0, 0};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    // |x| <= 127 (inv = 127 / absmax) and |x - xh| <= 1/2: both parts fit int8
                    const float x = qr[16 * s_ + 8 * half + order[e]] * inv;
                    const int xh = (int)rintf(x);
                    const int xl = (int)rintf((x - (float)xh) * 128.f);
                    h2[e >> 2] |= (uint32_t)(xh & 0xff) << (8 * (e & 3));
                    l2[e >> 2] |= (uint32_t)(xl & 0xff) << (8 * (e & 3));
                }
                hw[2 * half] = h2[0];
                hw[2 * half + 1] = h2[1];
                lw[2 * half] = l2[0];
                lw[2 * half + 1] = l2[1];
            }
            qh[s_] = u32x4{hw[0], hw[1], hw[2], hw[3]};
            ql[s_] = u32x4{lw[0], lw[1], lw[2], lw[3]};
        }
    }


    AttnState st;
    st.init();

    // The first two tile images landed while the query operand was built.
    if (n_tiles > 0) {
        wait_copies<0>();
        __syncthreads();
    }

    for (int ti = 0; ti < n_tiles; ++ti) {
        const int k0 = ti * kKT;
        const int nk = min(kKT, kv_end - k0);
        const uint8_t *tb = lds + (ti & 1) * kImBytes;
        const float s_unit = *reinterpret_cast<const float *>(tb + kImSk);  // score unit of this tile
        if (ti >= 1 && ti + 1 < n_tiles) issue_tile(ti + 1);  // tile 1 went out with tile 0
        // (every wave reaches the barrier at the end of the iteration)
        if (wave_active && (!causal || k0 <= pos_base + i0 + kPQ - 1)) {  // else: tile above this wave's diagonal
        // every key of the tile visible to all 16 positions of this wave: no mask
        const bool full = nk == kKT && (!causal || k0 + kKT - 1 <= pos_base + i0);

        // ---- S^T = K Q^T for 4 key blocks of 16 ----
        // s = hi.hi * 128 + hi.lo + lo.hi; the score proper is s * s_unit * sq.
        float s[16];
        if constexpr (KQ == kKqDtype) {
            // S^T = K Q^T on the q-dtype MFMA: four k-steps of 32 dims (half ks / 2 of the key row)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                f32x4 c = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const int ko = (ks >> 1) * (kKT * kKP) + 16 * b * kKP + ((ks & 1) ? koff1 : koff0);
                    const u32x4 kv = *reinterpret_cast<const u32x4 *>(tb + kImKhi + ko);
                    c = mfma_qk<DT>(kv, ks < 2 ? qh[ks] : ql[ks - 2], c);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) s[4 * b + i] = c[i];
            }
        } else
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            i32x4 chh = i32x4{0, 0, 0, 0}, cx = chh;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                // key 16b + col, piece 4ks + g (the swizzle term of key 16b + col is col & 7)
                const int ko = 16 * b * kKP + (ks ? koff1 : koff0);
                const u32x4 kh = *reinterpret_cast<const u32x4 *>(tb + kImKhi + ko);
                const u32x4 kl = *reinterpret_cast<const u32x4 *>(tb + kImKlo + ko);
                chh = mfma_i8(kh, qh[ks], chh);
                cx = mfma_i8(kh, ql[ks], cx);
                cx = mfma_i8(kl, qh[ks], cx);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) s[4 * b + i] = (float)((chh[i] << 7) + cx[i]);
        }
        if (!full) {  // causal and tile-end mask: key < min(k0 + nk, position + 1)
            const int lim = (causal ? min(k0 + nk, my_pos + 1) : k0 + nk) - (k0 + 4 * g);
#pragma unroll
            for (int j = 0; j < 16; ++j) s[j] = (16 * (j >> 2) + (j & 3)) < lim ? s[j] : -INFINITY;
        }
        // ---- online softmax and O^T += V'^T P'^T ----
        softmax_pv(st, s, s_unit, sq, *reinterpret_cast<const int *>(tb + kImVe), tb + kImVt, koff0, koff1,
                   *reinterpret_cast<const u32x4 *>(tb + ones_off));
        }
        wait_copies<0>();  // the next tile's image has landed
        __syncthreads();   // ... for every wave; this buffer is refilled next
    }
    if (!wave_active) return;

    // ---- epilogue: normalise, round to the q dtype, rotate back by R, round ----
    const float inv_l = attn_inv_l(st);
    if (i0 + col >= T) return;
    uint16_t *orow = reinterpret_cast<uint16_t *>(a.out) + (int64_t)(q0 + i0 + col) * a.o_st + (int64_t)hq * a.o_sh;
    store_rotated<DT>(st, inv_l, orow, a.R, a.rot_block, g);
}

template <int DT, int KQ>
static void launch_pack(const PrefillArgs &a, int64_t num_seqs, hipStream_t st) {
    dim3 grid((unsigned)a.max_tiles, (unsigned)a.H, (unsigned)num_seqs);
    hipLaunchKernelGGL((prefill_pack_kernel<DT, KQ>), grid, dim3(256), 0, st, a);
}

template <int DT, int KQ>
static void launch_attn(const PrefillArgs &a, int64_t num_seqs, int64_t max_q_len, int nwaves, hipStream_t st) {
    const size_t lds = 2 * (size_t)kImBytes;
    const int64_t nx = a.flat ? ((max_q_len + kPQ - 1) / kPQ * a.G + nwaves - 1) / nwaves : (max_q_len + a.qb - 1) / a.qb;
    dim3 grid((unsigned)nx, (unsigned)a.H, (unsigned)num_seqs);
    hipLaunchKernelGGL((prefill_attn_kernel<DT, KQ>), grid, dim3(64 * nwaves), lds, st, a);
}

static int64_t prefill_tiles(int64_t max_seq_len) { return (max_seq_len + kKT - 1) / kKT; }

}  // namespace rq

using namespace rq;

extern "C" int64_t rq_int8_prefill_workspace_bytes(int64_t num_seqs, int32_t num_kv_heads, int64_t max_seq_len) {
    if (num_seqs <= 0 || num_kv_heads <= 0 || max_seq_len <= 0) return 0;
    return num_seqs * num_kv_heads * prefill_tiles(max_seq_len) * kImBytes;
}

namespace {

// The two entry points share the kernels; kq selects the K operand (int8 hi/lo, or
// rounded to the q dtype with V rounded likewise) and causal the mask.
int prefill_call(int kq, int causal, const void *q, int32_t dtype, int64_t total_q, int32_t num_q_heads,
                 int64_t q_stride_tok, int64_t q_stride_head, const int32_t *cu_seqlens_q, int64_t num_seqs,
                 int64_t max_q_len, const uint8_t *kv_cache, int64_t num_blocks, int32_t block_size,
                 int64_t stride_block, int64_t stride_token, int32_t num_kv_heads, int32_t head_dim,
                 int32_t index_layout, const int32_t *block_table, int64_t max_blocks, int64_t bt_stride_seq,
                 const int32_t *seq_lens, int64_t max_seq_len, const float *k_centroids, int32_t n_k_centroids,
                 const float *v_centroids, int32_t n_v_centroids, const float *rotation, int32_t rot_block,
                 float sm_scale, void *out, int64_t out_stride_tok, int64_t out_stride_head, void *workspace,
                 int64_t workspace_bytes, void *stream) {
    RQ_CHECK_ARG(dtype == RQ_DTYPE_BF16 || dtype == RQ_DTYPE_F16, "prefill dtype must be f16 or bf16");
    RQ_CHECK_ARG(head_dim == kPD, "head_dim %d unsupported (only %d)", head_dim, kPD);
    RQ_CHECK_ARG(num_kv_heads >= 1 && num_q_heads % num_kv_heads == 0 && num_q_heads / num_kv_heads <= 16,
                 "num_q_heads %d / num_kv_heads %d must be an integer <= 16", num_q_heads, num_kv_heads);
    if (kq == kKqInt8)
        RQ_CHECK_ARG((n_k_centroids == 8 || n_k_centroids == 16) && (n_v_centroids == 8 || n_v_centroids == 16),
                     "centroid counts must be 8 or 16");
    else
        RQ_CHECK_ARG(n_k_centroids >= 1 && n_k_centroids <= 16 && n_v_centroids >= 1 && n_v_centroids <= 16,
                     "centroid counts must be 1..16");
    RQ_CHECK_ARG(rot_block == 2 || rot_block == 4, "rot_block %d must be 2 or 4", rot_block);
    RQ_CHECK_ARG(num_seqs >= 0 && total_q >= 0 && max_q_len >= 0 && block_size >= 1 && max_blocks >= 0 &&
                     max_seq_len >= 0,
                 "bad sizes");
    const int lrc = check_index_layout(index_layout, head_dim, n_k_centroids, n_v_centroids);
    if (lrc) return lrc;
    RQ_CHECK_ARG(stride_token % 4 == 0 && stride_block % 4 == 0 && ((uintptr_t)kv_cache % 4) == 0,
                 "cache slots must be 4-byte aligned");
    RQ_CHECK_ARG(((uintptr_t)q % 16) == 0 && (q_stride_tok * 2) % 16 == 0 && (q_stride_head * 2) % 16 == 0,
                 "q rows must be 16-byte aligned");
    RQ_CHECK_ARG(((uintptr_t)rotation % 16) == 0, "rotation must be 16-byte aligned");
    if (num_seqs == 0 || max_q_len == 0 || num_blocks == 0 || max_seq_len == 0) return RQ_OK;
    const int64_t need = rq_int8_prefill_workspace_bytes(num_seqs, num_kv_heads, max_seq_len);
    RQ_CHECK_SPACE(workspace_bytes >= need, "workspace too small: the call needs %lld bytes (got %lld)",
                   (long long)need, (long long)workspace_bytes);
    RQ_CHECK_ARG(workspace != nullptr && ((uintptr_t)workspace % 16) == 0, "workspace must be 16-byte aligned");
    PrefillArgs a{};
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
    a.HQ = num_q_heads;
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
    a.score_scale = sm_scale * kLog2eP;
    a.causal = causal != 0;
    a.npg = std::max(1, 8 / a.G);
    a.qb = kPQ * a.npg;
    // GQA groups of 3, 5, 6 or 7 query heads: G * npg waves (6, 5, 6, 7) per workgroup
    // would load a CU's four SIMDs unevenly (two 7-wave workgroups: 4, 4, 3, 3 waves,
    // and each tile's barrier paces a workgroup by its busiest SIMD); they take
    // workgroups of 8 waves over the flattened (position group, query head) units.
    a.flat = a.G < 8 && (a.G * a.npg) % 4 != 0;
    a.max_tiles = prefill_tiles(max_seq_len);
    a.ws = static_cast<uint8_t *>(workspace);
    a.out = out;
    a.o_st = out_stride_tok;
    a.o_sh = out_stride_head;
    const int nwaves = a.flat ? 8 : a.G * a.npg;
    hipStream_t st = (hipStream_t)stream;
    const bool bf = dtype == RQ_DTYPE_BF16;
    if (kq == kKqInt8) {
        if (bf) launch_pack<RQ_DTYPE_BF16, kKqInt8>(a, num_seqs, st);
        else launch_pack<RQ_DTYPE_F16, kKqInt8>(a, num_seqs, st);
    } else {
        if (bf) launch_pack<RQ_DTYPE_BF16, kKqDtype>(a, num_seqs, st);
        else launch_pack<RQ_DTYPE_F16, kKqDtype>(a, num_seqs, st);
    }
    int rc = check_launch("prefill_pack_kernel");
    if (rc) return rc;
    if (kq == kKqInt8) {
        if (bf) launch_attn<RQ_DTYPE_BF16, kKqInt8>(a, num_seqs, max_q_len, nwaves, st);
        else launch_attn<RQ_DTYPE_F16, kKqInt8>(a, num_seqs, max_q_len, nwaves, st);
    } else {
        if (bf) launch_attn<RQ_DTYPE_BF16, kKqDtype>(a, num_seqs, max_q_len, nwaves, st);
        else launch_attn<RQ_DTYPE_F16, kKqDtype>(a, num_seqs, max_q_len, nwaves, st);
    }
    return check_launch("prefill_attn_kernel");
}

}  // namespace

extern "C" int rq_int8_prefill(const void *q, int32_t dtype, int64_t total_q, int32_t num_q_heads,
                               int64_t q_stride_tok, int64_t q_stride_head, const int32_t *cu_seqlens_q,
                               int64_t num_seqs, int64_t max_q_len, const uint8_t *kv_cache, int64_t num_blocks,
                               int32_t block_size, int64_t stride_block, int64_t stride_token, int32_t num_kv_heads,
                               int32_t head_dim, int32_t index_layout, const int32_t *block_table,
                               int64_t max_blocks, int64_t bt_stride_seq, const int32_t *seq_lens,
                               int64_t max_seq_len,
                               const float *k_centroids, int32_t n_k_centroids, const float *v_centroids,
                               int32_t n_v_centroids, const float *rotation, int32_t rot_block, float sm_scale,
                               void *out, int64_t out_stride_tok, int64_t out_stride_head, void *workspace,
                               int64_t workspace_bytes, void *stream) {
    return prefill_call(kKqInt8, 1, q, dtype, total_q, num_q_heads, q_stride_tok, q_stride_head, cu_seqlens_q,
                        num_seqs, max_q_len, kv_cache, num_blocks, block_size, stride_block, stride_token,
                        num_kv_heads, head_dim, index_layout, block_table, max_blocks, bt_stride_seq, seq_lens,
                        max_seq_len, k_centroids, n_k_centroids, v_centroids, n_v_centroids, rotation, rot_block,
                        sm_scale, out, out_stride_tok, out_stride_head, workspace, workspace_bytes, stream);
}

extern "C" int64_t rq_paged_prefill_workspace_bytes(int64_t num_seqs, int32_t num_kv_heads, int64_t max_seq_len) {
    return rq_int8_prefill_workspace_bytes(num_seqs, num_kv_heads, max_seq_len);
}

extern "C" int rq_paged_prefill(const void *q, int32_t dtype, int64_t total_q, int32_t num_q_heads,
                                int64_t q_stride_tok, int64_t q_stride_head, const int32_t *cu_seqlens_q,
                                int64_t num_seqs, int64_t max_q_len, int32_t causal, const uint8_t *kv_cache,
                                int64_t num_blocks, int32_t block_size, int64_t stride_block, int64_t stride_token,
                                int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                                const int32_t *block_table, int64_t max_blocks, int64_t bt_stride_seq,
                                const int32_t *seq_lens, int64_t max_seq_len, const float *k_centroids,
                                int32_t n_k_centroids, const float *v_centroids, int32_t n_v_centroids,
                                const float *rotation, int32_t rot_block, float sm_scale, void *out,
                                int64_t out_stride_tok, int64_t out_stride_head, void *workspace,
                                int64_t workspace_bytes, void *stream) {
    return prefill_call(kKqDtype, causal, q, dtype, total_q, num_q_heads, q_stride_tok, q_stride_head, cu_seqlens_q,
                        num_seqs, max_q_len, kv_cache, num_blocks, block_size, stride_block, stride_token,
                        num_kv_heads, head_dim, index_layout, block_table, max_blocks, bt_stride_seq, seq_lens,
                        max_seq_len, k_centroids, n_k_centroids, v_centroids, n_v_centroids, rotation, rot_block,
                        sm_scale, out, out_stride_tok, out_stride_head, workspace, workspace_bytes, stream);
}
