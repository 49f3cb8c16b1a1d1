// Fused paged decode attention over the packed RotorQuant cache (gfx950).
//
// Replaces fused_paged_rq_decode (src/rotorquant_vllm/triton/fused_paged_rq_decode.py:214-312,
// kernel :32-206).  Same mathematics -- attention in the rotated space, with
// q_rot = bf16(q R^T), K/V = centroid[idx] * norm, exp2 online softmax, and
// out = bf16(bf16(out_rot) R) -- organised for CDNA4:
//
//   * grid (chunk, seq); a workgroup owns one chunk of a sequence's context
//     for ALL kv heads (one wave per kv head), so each token's contiguous
//     payload is read once and all GQA query heads of a kv head share it;
//   * Q K^T and P V run on v_mfma_f32_16x16x32_{bf16,f16}: the GQA group
//     (<= 16 query heads) is the 16-wide N side, tokens / head dims the M side;
//   * nibble -> 16-bit centroid lookups are register v_perm_b32 table lookups;
//     the K/V norms are factored out of the MFMA operands (applied to the
//     scores and to P), so the operands are raw centroids;
//   * split-KV: each chunk writes (m, l, acc) partials; a merge kernel
//     combines them (log-sum-exp), rounds, and rotates back by R.
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

#include "rq_common.h"

namespace rq {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;

constexpr int kD = 128;          // head_dim handled by this kernel
constexpr int kTile = 32;        // tokens per inner iteration
constexpr int kMaxWaves = 8;     // waves per workgroup (kv heads beyond 8 loop)
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

// Centroids (fp32) -> 16-bit table split in low / high bytes.
template <int DT>
__device__ __forceinline__ Table16 make_table(const float *c, int n) {
    Table16 t;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int e = 4 * w + i;
            uint32_t bits = e < n ? Elem<DT>::from_f32(c[e]) : 0u;
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
__device__ __forceinline__ u32x4 decode_row8(const Table16 &t, uint32_t x) {
    uint32_t odd = x & 0x0f0f0f0fu;          // e1 e3 e5 e7
    uint32_t even = (x >> 4) & 0x0f0f0f0fu;  // e0 e2 e4 e6
    uint2 e = lookup4<BITS>(t, even), o = lookup4<BITS>(t, odd);
    return u32x4{e.x, e.y, o.x, o.y};
}

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
    int chunk;          // tokens per workgroup (multiple of kTile)
    int max_chunks;
    int max_len;        // min(max_blocks * block_size, max_chunks * chunk): lengths are clamped to it
    int64_t num_blocks; // physical blocks; table entries outside [0, num_blocks) read block 0
    int wave_lds;       // per-wave LDS bytes: 512 + G * 256
    float *part_acc;    // [seq][chunk][HQ][D]
    float *part_ml;     // [seq][chunk][HQ][2]
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

// Registers of one 32-token tile for one kv head (loaded one tile ahead).
struct TileRegs {
    uint4 kw[2];      // K indices: token 16j + (lane & 15), bytes 16g .. 16g+15 of the head
    uint32_t vw[8];   // V indices: dword (lane & 15) of tokens 4g+i (i < 4) and 16+4g+(i-4)
    float nrm;        // lane < 32: K norm * score_scale of token lane; else V norm of token lane-32
                      // (zero for tokens past the end)
};

template <int DT, int KB, int VB>
__global__ __launch_bounds__(512) void decode_kernel(DecodeArgs a) {
    const int chunk_id = blockIdx.x;
    const int64_t seq = blockIdx.y;
    const int L = min(a.seq_lens[seq], a.max_len);
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;    // k-group / row-group
    const int col = lane & 15;  // MFMA column (query head inside the GQA group) / row

    const int t_begin = chunk_id * a.chunk;
    if (t_begin >= L) return;
    const int n_tok = min(L - t_begin, a.chunk);
    const SlotLayout SL(a.H, kD);

    extern __shared__ __align__(16) uint8_t lds[];
    // per wave: 32 token byte offsets | 64 norms | G x 128 q_rot (16-bit)
    uint8_t *wbase = lds + wave * a.wave_lds;
    uint64_t *woff = reinterpret_cast<uint64_t *>(wbase);
    float *wnorm = reinterpret_cast<float *>(wbase + 256);
    uint16_t *wq = reinterpret_cast<uint16_t *>(wbase + 512);
    const int32_t *bt_row = a.bt + seq * a.bt_ss;

    const int nwaves = blockDim.x >> 6;
    for (int h = wave; h < a.H; h += nwaves) {
        // ---- rotated queries of this wave's GQA group: q_rot = q R^T, rounded to the q dtype ----
        for (int idx = lane; idx < a.G * kD; idx += 64) {
            int qh = idx / kD, j = idx - qh * kD;
            const uint16_t *qrow = reinterpret_cast<const uint16_t *>(a.q) + seq * a.q_ss + (int64_t)(h * a.G + qh) * a.q_sh;
            int k0 = (j / a.rot_block) * a.rot_block;
            float acc = 0.f;
            for (int i = 0; i < a.rot_block; ++i)
                acc = __builtin_fmaf(Elem<DT>::to_f32(qrow[k0 + i]), a.R[j * kD + k0 + i], acc);
            wq[qh * kD + j] = (uint16_t)Elem<DT>::from_f32(acc);
        }
        __builtin_amdgcn_wave_barrier();

        // Q^T operand: lane (g, col) for dim chunk c holds dims 32g + 8c + {0,2,4,6,1,3,5,7}.
        // The MFMA runs in fp16 for any query dtype: the dtype-rounded q_rot is
        // scaled by 2^qexp (exact) so its largest element sits in [2^14, 2^15).
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
        qmax = fmaxf(qmax, __shfl_xor(qmax, 16));
        qmax = fmaxf(qmax, __shfl_xor(qmax, 32));
        const int qexp = qmax > 0.f ? 141 - (int)((__float_as_uint(qmax) >> 23) & 0xffu) : 0;  // 14 - floor(log2 qmax)
        const float qinv = ldexpf(1.f, -qexp);
        u32x4 qop[4];
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

        const Table16 tk = make_table<RQ_DTYPE_F16>(a.kc, a.nkc);
        const Table16 tv = make_table<RQ_DTYPE_F16>(a.vc, a.nvc);

        f32x4 acc[8];
    #pragma unroll
        for (int m = 0; m < 8; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
        float m_run = -INFINITY;  // running max (log2 domain) for query head `col`
        float l_run = 0.f;        // this lane's partial sum of p
        int e_run = -126;         // P operand = p * v_norm * 2^-e_run <= 1 (fp16); acc carries the same scale

        const uint8_t *cache = a.cache;
        const int k_idx = SL.k_idx + h * 64;
        const int v_idx = SL.v_idx + h * 64;
        const int k_norm = SL.k_norm + 4 * h;
        const int v_norm = SL.v_norm + 4 * h;
        const int my_tt = lane & 31;

        // Issue the loads of the tile starting at t0.  Tokens past the end read
        // slot 0 of block 0 (always mapped) and get a zero norm.
        auto load_tile = [&](int t0) {
            TileRegs r;
            const int valid = n_tok - t0;
            uint64_t my_off = 0;
            const bool ok = my_tt < valid;
            if (ok) {
                int pos = t_begin + t0 + my_tt;
                int lb, off;
                if (a.bs_shift >= 0) {
                    lb = pos >> a.bs_shift;
                    off = pos & (a.block_size - 1);
                } else {
                    lb = pos / a.block_size;
                    off = pos - lb * a.block_size;
                }
                int64_t phys = bt_row[lb];
                phys = (phys < 0 || phys >= a.num_blocks) ? 0 : phys;
                my_off = (uint64_t)(phys * a.stride_block + (int64_t)off * a.stride_token);
            }
            if (lane < 32) woff[lane] = my_off;
            __builtin_amdgcn_wave_barrier();
            const uint64_t ok0 = woff[col], ok1 = woff[16 + col];
            r.kw[0] = *reinterpret_cast<const uint4 *>(cache + ok0 + k_idx + 16 * g);
            r.kw[1] = *reinterpret_cast<const uint4 *>(cache + ok1 + k_idx + 16 * g);
            const ulonglong2 va = *reinterpret_cast<const ulonglong2 *>(woff + 4 * g);
            const ulonglong2 vb = *reinterpret_cast<const ulonglong2 *>(woff + 4 * g + 2);
            const ulonglong2 vc = *reinterpret_cast<const ulonglong2 *>(woff + 16 + 4 * g);
            const ulonglong2 vd = *reinterpret_cast<const ulonglong2 *>(woff + 16 + 4 * g + 2);
            const uint64_t vo[8] = {va.x, va.y, vb.x, vb.y, vc.x, vc.y, vd.x, vd.y};
    #pragma unroll
            for (int i = 0; i < 8; ++i) r.vw[i] = *reinterpret_cast<const uint32_t *>(cache + vo[i] + v_idx + 4 * col);
            float nv = *reinterpret_cast<const float *>(cache + my_off + (lane < 32 ? k_norm : v_norm));
            nv = lane < 32 ? nv * a.score_scale : nv;
            r.nrm = ok ? nv : 0.f;
            __builtin_amdgcn_wave_barrier();
            return r;
        };

        TileRegs cur = load_tile(0);
        for (int t0 = 0; t0 < n_tok; t0 += kTile) {
            const int valid = n_tok - t0;
            TileRegs nxt;
            if (t0 + kTile < n_tok) nxt = load_tile(t0 + kTile);

            // largest V norm of the tile (lanes 32..63) -> power-of-two scale of P
            float nvm = lane >= 32 ? cur.nrm : 0.f;
    #pragma unroll
            for (int o = 1; o < 32; o <<= 1) nvm = fmaxf(nvm, __shfl_xor(nvm, o));
            const int e_tile = (int)((__float_as_uint(__shfl(nvm, 32)) >> 23) & 0xffu) - 126;  // 2^e_tile > max norm
            if (e_tile > e_run) {
                const float f = ldexpf(1.f, e_run - e_tile);
    #pragma unroll
                for (int m = 0; m < 8; ++m) acc[m] *= f;
                e_run = e_tile;
            }
            wnorm[lane] = lane < 32 ? cur.nrm : ldexpf(cur.nrm, -e_run);
            __builtin_amdgcn_wave_barrier();

            // ---- S^T = K Q^T ----------------------------------------------------
            f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = s0;
            {
                const uint32_t k0w[4] = {cur.kw[0].x, cur.kw[0].y, cur.kw[0].z, cur.kw[0].w};
                const uint32_t k1w[4] = {cur.kw[1].x, cur.kw[1].y, cur.kw[1].z, cur.kw[1].w};
    #pragma unroll
                for (int c = 0; c < 4; ++c) {
                    s0 = mfma<RQ_DTYPE_F16>(decode_row8<KB>(tk, k0w[c]), qop[c], s0);
                    s1 = mfma<RQ_DTYPE_F16>(decode_row8<KB>(tk, k1w[c]), qop[c], s1);
                }
            }
            // ---- scale by K norm, mask, online softmax ---------------------------
            const float4 nk0 = *reinterpret_cast<const float4 *>(wnorm + 4 * g);
            const float4 nk1 = *reinterpret_cast<const float4 *>(wnorm + 16 + 4 * g);
            const float4 nv0 = *reinterpret_cast<const float4 *>(wnorm + 32 + 4 * g);
            const float4 nv1 = *reinterpret_cast<const float4 *>(wnorm + 48 + 4 * g);
            // undo the query's power-of-two scale (per query head = per lane column)
            float s[8] = {s0.x * nk0.x * qinv, s0.y * nk0.y * qinv, s0.z * nk0.z * qinv, s0.w * nk0.w * qinv,
                          s1.x * nk1.x * qinv, s1.y * nk1.y * qinv, s1.z * nk1.z * qinv, s1.w * nk1.w * qinv};
            if (valid < kTile) {
    #pragma unroll
                for (int i = 0; i < 8; ++i) {
                    int tt = (i < 4) ? 4 * g + i : 16 + 4 * g + (i - 4);
                    s[i] = tt < valid ? s[i] : -INFINITY;
                }
            }
            float tmax = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            if (__any(tmax > m_run)) {
                const float m_new = fmaxf(m_run, tmax);
                const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // m_run = -inf on the first tile -> 0
    #pragma unroll
                for (int m = 0; m < 8; ++m) acc[m] *= alpha;
                l_run *= alpha;
                m_run = m_new;
            }
            float p[8];
    #pragma unroll
            for (int i = 0; i < 8; ++i) {
                p[i] = __builtin_amdgcn_exp2f(s[i] - m_run);
                l_run += p[i];
            }
            u32x4 pop;
            pop.x = pack2<RQ_DTYPE_F16>(p[0] * nv0.x, p[1] * nv0.y);
            pop.y = pack2<RQ_DTYPE_F16>(p[2] * nv0.z, p[3] * nv0.w);
            pop.z = pack2<RQ_DTYPE_F16>(p[4] * nv1.x, p[5] * nv1.y);
            pop.w = pack2<RQ_DTYPE_F16>(p[6] * nv1.z, p[7] * nv1.w);

            // ---- O^T += V^T P^T ---------------------------------------------------
            // Byte-transpose the 8 tokens' dwords: Ga[j] = byte j of tokens 0..3,
            // Gb[j] = byte j of tokens 4..7; then split nibbles per head dim.
            const uint32_t *vw = cur.vw;
            uint32_t A01 = perm(vw[1], vw[0], 0x05010400u), B01 = perm(vw[1], vw[0], 0x07030602u);
            uint32_t A23 = perm(vw[3], vw[2], 0x05010400u), B23 = perm(vw[3], vw[2], 0x07030602u);
            uint32_t A45 = perm(vw[5], vw[4], 0x05010400u), B45 = perm(vw[5], vw[4], 0x07030602u);
            uint32_t A67 = perm(vw[7], vw[6], 0x05010400u), B67 = perm(vw[7], vw[6], 0x07030602u);
            uint32_t Ga[4] = {perm(A23, A01, 0x05040100u), perm(A23, A01, 0x07060302u), perm(B23, B01, 0x05040100u),
                              perm(B23, B01, 0x07060302u)};
            uint32_t Gb[4] = {perm(A67, A45, 0x05040100u), perm(A67, A45, 0x07060302u), perm(B67, B45, 0x05040100u),
                              perm(B67, B45, 0x07060302u)};
    #pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint2 ha = lookup4<VB>(tv, (Ga[j] >> 4) & 0x0f0f0f0fu), hb = lookup4<VB>(tv, (Gb[j] >> 4) & 0x0f0f0f0fu);
                uint2 la = lookup4<VB>(tv, Ga[j] & 0x0f0f0f0fu), lb = lookup4<VB>(tv, Gb[j] & 0x0f0f0f0fu);
                acc[2 * j] = mfma<RQ_DTYPE_F16>(u32x4{ha.x, ha.y, hb.x, hb.y}, pop, acc[2 * j]);          // dim 8r + 2j
                acc[2 * j + 1] = mfma<RQ_DTYPE_F16>(u32x4{la.x, la.y, lb.x, lb.y}, pop, acc[2 * j + 1]);  // dim 8r + 2j + 1
            }
            __builtin_amdgcn_wave_barrier();
            cur = nxt;
        }

        // ---- partials ------------------------------------------------------------
        l_run += __shfl_xor(l_run, 16);
        l_run += __shfl_xor(l_run, 32);
        if (col < a.G) {
            const int hq = h * a.G + col;
            const int64_t pidx = (seq * a.max_chunks + chunk_id) * a.HQ + hq;
            float *pa = a.part_acc + pidx * kD;
            // acc[m][i] * 2^e_run = O[col][8 * (4g + i) + m]
            const float es = ldexpf(1.f, e_run);
    #pragma unroll
            for (int i = 0; i < 4; ++i) {
                float4 lo = make_float4(acc[0][i] * es, acc[1][i] * es, acc[2][i] * es, acc[3][i] * es);
                float4 hi = make_float4(acc[4][i] * es, acc[5][i] * es, acc[6][i] * es, acc[7][i] * es);
                float4 *dst = reinterpret_cast<float4 *>(pa + 8 * (4 * g + i));
                dst[0] = lo;
                dst[1] = hi;
            }
            if (g == 0) {
                a.part_ml[pidx * 2] = m_run;
                a.part_ml[pidx * 2 + 1] = l_run;
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// Merge the chunk partials of (seq, query head): log-sum-exp over chunks, round
// to the query dtype (the reference's out_rot, fused_paged_rq_decode.py:201-206),
// rotate back by R in fp32 and round again (:308).  One wave per query head,
// two head dims per lane; the chunk loop issues its loads four at a time.
template <int DT>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    const int64_t seq = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int hq = blockIdx.x * 4 + wave;
    __shared__ float orot_all[4][kD];
    float *orot = orot_all[wave];
    if (hq >= a.HQ) return;
    const int L = min(a.seq_lens[seq], a.max_len);
    const int nch = L > 0 ? (L + a.chunk - 1) / a.chunk : 0;
    const float *ml = a.part_ml + (seq * a.max_chunks) * (int64_t)a.HQ * 2 + hq * 2;
    const float *pa = a.part_acc + (seq * a.max_chunks) * (int64_t)a.HQ * kD + hq * kD;
    const int64_t cs_ml = (int64_t)a.HQ * 2, cs_acc = (int64_t)a.HQ * kD;
    float M = -INFINITY;
    for (int c = 0; c < nch; ++c) M = fmaxf(M, ml[c * cs_ml]);
    float lsum = 0.f, o0 = 0.f, o1 = 0.f;
    int c = 0;
    for (; c + 4 <= nch; c += 4) {
        float w[4], l[4];
        float2 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            w[u] = ml[(c + u) * cs_ml];
            l[u] = ml[(c + u) * cs_ml + 1];
            v[u] = reinterpret_cast<const float2 *>(pa + (c + u) * cs_acc)[lane];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float e = exp2f(w[u] - M);
            lsum += e * l[u];
            o0 += e * v[u].x;
            o1 += e * v[u].y;
        }
    }
    for (; c < nch; ++c) {
        const float e = exp2f(ml[c * cs_ml] - M);
        lsum += e * ml[c * cs_ml + 1];
        const float2 v = reinterpret_cast<const float2 *>(pa + c * cs_acc)[lane];
        o0 += e * v.x;
        o1 += e * v.y;
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
        for (int i = 0; i < a.rot_block; ++i) r = __builtin_fmaf(orot[k0 + i], a.R[(k0 + i) * kD + d], r);
        packed |= Elem<DT>::from_f32(r) << (16 * e);
    }
    reinterpret_cast<uint32_t *>(dst)[lane] = packed;
}

static int pick_chunk(int64_t num_seqs, int64_t max_seq_len) {
    int64_t c = 256;
    while (c < 16384 && num_seqs * ((max_seq_len + c - 1) / c) > 4096) c *= 2;
    return (int)c;
}

template <int DT, int KB, int VB>
static void launch_decode(const DecodeArgs &a, int64_t num_seqs, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL((decode_kernel<DT, KB, VB>), dim3(a.max_chunks, (unsigned)num_seqs),
                       dim3(64 * std::min(a.H, kMaxWaves)), lds, st, a);
}

template <int DT>
static void launch_decode_bits(const DecodeArgs &a, int64_t num_seqs, size_t lds, int kb, int vb, hipStream_t st) {
    if (kb == 3 && vb == 3) launch_decode<DT, 3, 3>(a, num_seqs, lds, st);
    else if (kb == 3) launch_decode<DT, 3, 4>(a, num_seqs, lds, st);
    else if (vb == 3) launch_decode<DT, 4, 3>(a, num_seqs, lds, st);
    else launch_decode<DT, 4, 4>(a, num_seqs, lds, st);
}

}  // namespace rq

using namespace rq;

extern "C" int64_t rq_fused_decode_workspace_bytes(int64_t num_seqs, int32_t num_q_heads, int32_t head_dim,
                                                   int64_t max_seq_len) {
    int chunk = pick_chunk(num_seqs, max_seq_len);
    int64_t max_chunks = (max_seq_len + chunk - 1) / chunk;
    if (max_chunks < 1) max_chunks = 1;
    int64_t n = num_seqs * max_chunks * num_q_heads;
    return n * ((int64_t)head_dim + 2) * (int64_t)sizeof(float) + 256;
}

extern "C" int rq_fused_decode(const void *q, int32_t dtype, int64_t num_seqs, int32_t num_q_heads,
                               int64_t q_stride_seq, int64_t q_stride_head, const uint8_t *kv_cache,
                               int64_t num_blocks, int32_t block_size, int64_t stride_block, int64_t stride_token,
                               int32_t num_kv_heads, int32_t head_dim, const int32_t *block_table, int64_t max_blocks,
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
    RQ_CHECK_ARG(max_seq_len <= max_blocks * block_size, "max_seq_len exceeds block table capacity");
    RQ_CHECK_ARG(stride_token % 16 == 0 && stride_block % 16 == 0 && ((uintptr_t)kv_cache % 16) == 0,
                 "cache slots must be 16-byte aligned");
    RQ_CHECK_ARG(((uintptr_t)q % 16) == 0 && (q_stride_head * 2) % 16 == 0 && (q_stride_seq * 2) % 16 == 0,
                 "q rows must be 16-byte aligned");
    if (num_seqs == 0) return RQ_OK;
    RQ_CHECK_ARG(workspace_bytes >= rq_fused_decode_workspace_bytes(num_seqs, num_q_heads, head_dim, max_seq_len),
                 "workspace too small");
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
    a.chunk = pick_chunk(num_seqs, max_seq_len);
    int64_t max_chunks = (max_seq_len + a.chunk - 1) / a.chunk;
    a.max_chunks = (int)(max_chunks < 1 ? 1 : max_chunks);
    a.part_acc = reinterpret_cast<float *>(workspace);
    a.part_ml = a.part_acc + num_seqs * (int64_t)a.max_chunks * num_q_heads * kD;
    a.num_blocks = num_blocks;
    a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
    a.wave_lds = 512 + a.G * kD * 2;
    a.max_len = num_blocks > 0 ? (int)std::min<int64_t>(max_blocks * block_size, (int64_t)a.max_chunks * a.chunk) : 0;
    a.out = out;
    a.o_ss = out_stride_seq;
    a.o_sh = out_stride_head;
    const int nwaves = std::min(a.H, kMaxWaves);
    size_t lds = (size_t)nwaves * a.wave_lds;
    int kb = n_k_centroids == 8 ? 3 : 4, vb = n_v_centroids == 8 ? 3 : 4;
    if (a.max_len > 0) {
        if (dtype == RQ_DTYPE_BF16) launch_decode_bits<RQ_DTYPE_BF16>(a, num_seqs, lds, kb, vb, st);
        else launch_decode_bits<RQ_DTYPE_F16>(a, num_seqs, lds, kb, vb, st);
        int rc = check_launch("decode_kernel");
        if (rc) return rc;
    }
    dim3 mgrid((num_q_heads + 3) / 4, (unsigned)num_seqs);
    if (dtype == RQ_DTYPE_BF16) hipLaunchKernelGGL(decode_merge_kernel<RQ_DTYPE_BF16>, mgrid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(decode_merge_kernel<RQ_DTYPE_F16>, mgrid, dim3(256), 0, st, a);
    return check_launch("decode_merge_kernel");
}
