/*
 * rq_oracle.c -- TEST INFRASTRUCTURE ONLY.  CPU restatement of the reference's
 * compress / decompress arithmetic, used as the parity checker by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg.  Nothing in the
 * product (rotorquant-vllm_amd/) may call it.
 *
 * Follows (tpurtell/rotorquant-vllm):
 *   rqo_compress   : src/rotorquant_vllm/triton/isoquant_compress.py:161-190
 *                    (identical planar path: planarquant_compress.py:157-186)
 *   rqo_decompress : src/rotorquant_vllm/triton/isoquant_decompress.py:103-133
 *                    (identical planar path: planarquant_decompress.py:104-133)
 *
 * The reference expresses these with torch CPU ops whose rounding order is a
 * library property.  The orders restated here were fixed by black-box
 * comparison against torch 2.10 / MKL 2024.2 on AVX-512 (tests/golden holds
 * the vectors that pin them):
 *   torch.norm(x, dim=-1) : eight lane sums s_v = fma(x[8k+v], x[8k+v], s_v)
 *                           over k in order, then ((s0+s1)+s2)+...+s7, sqrt.
 *   normalized @ R^T      : for a block-diagonal R^T and M >= 2 rows, each
 *                           output is an fma chain over its block in
 *                           increasing k, starting from the first product.
 *                           (M == 1 takes MKL's gemv path, whose order is not
 *                           restated; callers keep M >= 2.)
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; fmaf from libm).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { RQO_F16 = 0, RQO_BF16 = 1, RQO_F32 = 2 };

static float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do {
                man <<= 1;
                ++e;
            } while (!(man & 0x400));
            man &= 0x3ff;
            u = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        u = sign | 0x7f800000u | (man << 13);
    } else {
        u = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float load_elem(const void *x, int dtype, int64_t i) {
    switch (dtype) {
        case RQO_F16: return f16_to_f32(((const uint16_t *)x)[i]);
        case RQO_BF16: return bf16_to_f32(((const uint16_t *)x)[i]);
        default: return ((const float *)x)[i];
    }
}

/* torch.norm over one row (isoquant_compress.py:174). */
float rqo_row_norm(const float *x, int D) {
    float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int k = 0; k < D / 8; ++k)
        for (int v = 0; v < 8; ++v) s[v] = fmaf(x[8 * k + v], x[8 * k + v], s[v]);
    float sum = s[0];
    for (int v = 1; v < 8; ++v) sum = sum + s[v];
    return sqrtf(sum);
}

/*
 * Compress n_rows rows (isoquant_compress.py:172-190).
 * rt_even / rt_odd: D x D/2 row-major even / odd columns of R^T.
 * blk: diagonal block width of R^T (2, 4, ..., or D for a dense product).
 * ties (optional, n_rows * D bytes): 1 where the rotated coordinate equals a
 * boundary exactly (the place where the reference's CPU and GPU paths
 * disagree: bucketize puts the tie in the lower bucket, the Triton kernel's
 * `x >= b` count in the upper one).
 * Returns the number of ties.
 */
int64_t rqo_compress(const void *x, int dtype, int64_t n_rows, int D, const float *rt_even, const float *rt_odd,
                     int blk, const float *bounds, int nb, uint8_t *packed, float *norms, uint8_t *ties) {
    float row[512], xn[512];
    int64_t n_ties = 0;
    const int half = D / 2;
    for (int64_t r = 0; r < n_rows; ++r) {
        for (int k = 0; k < D; ++k) row[k] = load_elem(x, dtype, r * D + k);
        float n = rqo_row_norm(row, D);
        norms[r] = n;                         /* stored without the eps (:190) */
        float den = n + 1e-10f;               /* :175, fp32 add */
        for (int k = 0; k < D; ++k) xn[k] = row[k] / den;
        for (int j = 0; j < D; j += 2) {
            int idx2[2];
            for (int e = 0; e < 2; ++e) {
                int jj = j + e;
                const float *colm = (jj & 1) ? rt_odd : rt_even;
                int k0 = (jj / blk) * blk;
                float acc = xn[k0] * colm[(int64_t)k0 * half + (jj >> 1)];
                for (int i = 1; i < blk; ++i) acc = fmaf(xn[k0 + i], colm[(int64_t)(k0 + i) * half + (jj >> 1)], acc);
                int idx = 0, tie = 0;
                for (int b = 0; b < nb; ++b) {
                    if (bounds[b] < acc) ++idx;
                    if (bounds[b] == acc) tie = 1;
                }
                if (idx > 15) idx = 15; /* clamp(0, 15) (:185) */
                idx2[e] = idx;
                if (ties) ties[r * D + jj] = (uint8_t)tie;
                n_ties += tie;
            }
            packed[r * half + j / 2] = (uint8_t)((idx2[0] << 4) | idx2[1]);
        }
    }
    return n_ties;
}

/*
 * Decompress (isoquant_decompress.py:114-133): out[2j] = c[hi] * n,
 * out[2j+1] = c[lo] * n in fp32; the caller applies the dtype cast.
 * Nibbles >= n_c read 0.0 (the reference raises IndexError there).
 */
void rqo_decompress(const uint8_t *packed, const float *norms, int64_t n_rows, int D, const float *cb, int n_c,
                    float *out) {
    const int half = D / 2;
    for (int64_t r = 0; r < n_rows; ++r) {
        float n = norms[r];
        for (int j = 0; j < half; ++j) {
            uint8_t p = packed[r * half + j];
            int hi = p >> 4, lo = p & 15;
            out[r * D + 2 * j] = (hi < n_c ? cb[hi] : 0.0f) * n;
            out[r * D + 2 * j + 1] = (lo < n_c ? cb[lo] : 0.0f) * n;
        }
    }
}

/*
 * Block-diagonal fp32 product out[r][j] = sum_k x[r][k] * M(k, j) over the
 * diagonal block of width blk that holds j, M(k, j) = M[k * sk + j * sj]:
 * the first product, then an fma chain in increasing k -- the order torch's
 * CPU fp32 matmul (MKL sgemm, M >= 2 rows) gives a block-diagonal operand
 * (entries outside the block are exact zeros and leave the sum unchanged).
 * Used for q_rot = q.float() @ R^T (sk = 1, sj = D; fused_paged_rq_decode.py:271)
 * and out = out_rot.float() @ R (sk = D, sj = 1; :308).
 */
void rqo_block_rotate(const float *x, int64_t rows, int D, const float *M, int64_t sk, int64_t sj, int blk,
                      float *out) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * D;
        for (int j = 0; j < D; ++j) {
            const int k0 = (j / blk) * blk;
            float acc = xr[k0] * M[k0 * sk + j * sj];
            for (int i = 1; i < blk; ++i) acc = fmaf(xr[k0 + i], M[(k0 + i) * sk + j * sj], acc);
            out[r * D + j] = acc;
        }
    }
}
