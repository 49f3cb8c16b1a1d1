// Compress kernels: norm -> divide -> block rotation -> Lloyd-Max bucketize ->
// nibble pack, bit-exact with the reference's CPU fallback
// (src/rotorquant_vllm/triton/isoquant_compress.py:161-190,
//  src/rotorquant_vllm/triton/planarquant_compress.py:157-186).
//
// Rounding contract (each step is one IEEE fp32 operation, no contraction;
// this TU is built with -ffp-contract=off):
//   norm  : eight partial sums s_v, s_v = fma(x[8k+v], x[8k+v], s_v) for
//           k = 0, 1, ... in order; then ((s_0 + s_1) + s_2) + ... + s_7;
//           n = sqrt(sum).  This is the order torch.norm's vectorised CPU
//           reduction uses (isoquant_compress.py:174).
//   divide: xn = x / (n + 1e-10f), correctly rounded (:175).
//   rotate: r_j = fma chain over the diagonal block of R^T in increasing k,
//           starting from xn[k0] * RT[k0][j] -- the order MKL's sgemm produces
//           for a block-diagonal R^T with M >= 2 rows (:182).
//   index : number of boundaries b with b < r_j (torch.bucketize right=False,
//           :184); pack byte j = (idx[2j] << 4) | idx[2j+1] (:187-188).
//
// Work split: one 64-lane wave owns 64 rows (one row = one (token, head) of K
// or V).  The rows are staged through LDS with coalesced 16-byte loads; each
// lane then reduces one row's norm in the fixed order above, and finally 16
// lanes per row each produce 8 indices (one packed dword).
#include "rq_common.h"

namespace rq {

constexpr int kRowsPerWave = 64;
constexpr int kMaxBounds = 15;
constexpr int kMaxD = 256;

// Where the rows come from and where their bytes go.
struct RowMap {
    // op-level mode (store == 0): row r at x + r * D, packed at r * D/2, norm at r.
    // store mode (store == 1): row r -> token t = r / (2H), kv = (r / H) & 1, head h = r % H.
    int store;
    const void *x;      // op mode input
    const void *key;    // store mode inputs
    const void *value;
    int64_t k_st, k_sh, v_st, v_sh;  // element strides
    uint8_t *packed;    // op mode outputs
    float *norms;
    const int64_t *slot_mapping;  // store mode outputs
    uint8_t *cache;
    int32_t block_size;
    int64_t num_slots;  // num_blocks * block_size; slots outside [0, num_slots) are skipped
    int64_t stride_block, stride_token;
    int32_t total_bytes;
    int32_t H;
};

// Byte address of the slot of row r's token (nullptr when the slot is < 0).
__device__ __forceinline__ uint8_t *slot_base(const RowMap &m, int64_t t) {
    int64_t s = m.slot_mapping[t];
    if (s < 0 || s >= m.num_slots) return nullptr;
    int64_t blk = s / m.block_size;
    int64_t off = s - blk * m.block_size;
    return m.cache + blk * m.stride_block + off * m.stride_token;
}

template <typename T>
__device__ __forceinline__ void load8(const uint8_t *lds, float (&x)[8]) {
    if constexpr (T::bytes == 2) {
        uint4 w = *reinterpret_cast<const uint4 *>(lds);
        uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = T::to_f32(ws[i] & 0xffffu);
            x[2 * i + 1] = T::to_f32(ws[i] >> 16);
        }
    } else {
        float4 a = *reinterpret_cast<const float4 *>(lds);
        float4 b = *reinterpret_cast<const float4 *>(lds + 16);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    }
}

template <int DT> struct Src;
template <> struct Src<RQ_DTYPE_F16> : Elem<RQ_DTYPE_F16> { static constexpr int bytes = 2; };
template <> struct Src<RQ_DTYPE_BF16> : Elem<RQ_DTYPE_BF16> { static constexpr int bytes = 2; };
template <> struct Src<RQ_DTYPE_F32> { static constexpr int bytes = 4; };

template <int DT, int BLK>
__global__ __launch_bounds__(64) void compress_kernel(RowMap m, int64_t n_rows, int D,
                                                      const float *__restrict__ rt_even,
                                                      const float *__restrict__ rt_odd,
                                                      const float *__restrict__ kbnd, int nkb,
                                                      const float *__restrict__ vbnd, int nvb) {
    using S = Src<DT>;
    constexpr int EB = S::bytes;
    const int lane = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * kRowsPerWave;
    const int row_bytes = D * EB;
    const int row_pitch = row_bytes + 16;  // +16 B keeps the per-row reads bank-conflict free
    const int chunks = row_bytes / 16;     // 16-byte pieces per row

    extern __shared__ __align__(16) uint8_t lds[];
    float *lds_norm = reinterpret_cast<float *>(lds + kRowsPerWave * row_pitch);

    // Boundaries: uniform loads, kept in registers.
    float kb[kMaxBounds], vb[kMaxBounds];
#pragma unroll
    for (int b = 0; b < kMaxBounds; ++b) {
        kb[b] = b < nkb ? kbnd[b] : 0.f;
        vb[b] = b < nvb ? vbnd[b] : 0.f;
    }

    // ---- phase 1: stage 64 rows in LDS with coalesced 16-byte loads -------
    const int total_chunks = kRowsPerWave * chunks;
    for (int c = lane; c < total_chunks; c += 64) {
        int rr = c / chunks, part = c - rr * chunks;
        int64_t r = row0 + rr;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (r < n_rows) {
            const uint8_t *src;
            if (!m.store) {
                src = reinterpret_cast<const uint8_t *>(m.x) + r * (int64_t)row_bytes;
            } else {
                int64_t t = r / (2 * m.H);
                int rem = (int)(r - t * 2 * m.H);
                bool is_v = rem >= m.H;
                int h = is_v ? rem - m.H : rem;
                int64_t off = is_v ? t * m.v_st + (int64_t)h * m.v_sh : t * m.k_st + (int64_t)h * m.k_sh;
                src = reinterpret_cast<const uint8_t *>(is_v ? m.value : m.key) + off * EB;
            }
            v = *reinterpret_cast<const uint4 *>(src + part * 16);
        }
        *reinterpret_cast<uint4 *>(lds + rr * row_pitch + part * 16) = v;
    }
    // Zero padding of every slot whose first row this wave owns.
    if (m.store) {
        int pay = SlotLayout(m.H, D).payload;
        int pad_words = (m.total_bytes - pay) / 4;
        for (int rr = 0; rr < kRowsPerWave; ++rr) {
            int64_t r = row0 + rr;
            if (r >= n_rows) break;
            if (r % (2 * m.H) != 0) continue;
            uint8_t *base = slot_base(m, r / (2 * m.H));
            if (base == nullptr) continue;
            for (int w = lane; w < pad_words; w += 64)
                reinterpret_cast<uint32_t *>(base + pay)[w] = 0u;
        }
    }
    __syncthreads();

    // ---- phase 2: one lane per row computes the norm in torch's order -----
    {
        float s[8];
#pragma unroll
        for (int v = 0; v < 8; ++v) s[v] = 0.f;
        const uint8_t *rowp = lds + lane * row_pitch;
        for (int k = 0; k < D / 8; ++k) {
            float x[8];
            load8<S>(rowp + k * 8 * EB, x);
#pragma unroll
            for (int v = 0; v < 8; ++v) s[v] = __builtin_fmaf(x[v], x[v], s[v]);
        }
        float sum = s[0];
#pragma unroll
        for (int v = 1; v < 8; ++v) sum = sum + s[v];
        float n = __builtin_sqrtf(sum);
        lds_norm[lane] = n;
        int64_t r = row0 + lane;
        if (r < n_rows) {
            if (!m.store) {
                m.norms[r] = n;
            } else {
                int64_t t = r / (2 * m.H);
                int rem = (int)(r - t * 2 * m.H);
                bool is_v = rem >= m.H;
                int h = is_v ? rem - m.H : rem;
                uint8_t *base = slot_base(m, t);
                SlotLayout L(m.H, D);
                if (base != nullptr)
                    *reinterpret_cast<float *>(base + (is_v ? L.v_norm : L.k_norm) + 4 * h) = n;
            }
        }
    }
    __syncthreads();

    // ---- phase 3: D/8 lanes per row, 8 coordinates per lane ---------------
    const int lanes_per_row = D / 8;
    const int rows_per_pass = 64 / lanes_per_row;
    const int part = lane % lanes_per_row;
    const int sub = lane / lanes_per_row;
    const int half = D / 2;
    // R^T entries for this lane's 8 outputs: RT[k][j] for k in j's block.
    float rt[8][BLK];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        int j = part * 8 + e;
        int k0 = (j / BLK) * BLK;
        const float *col = (j & 1) ? rt_odd : rt_even;
#pragma unroll
        for (int i = 0; i < BLK; ++i) rt[e][i] = col[(int64_t)(k0 + i) * half + (j >> 1)];
    }
    for (int p0 = 0; p0 < kRowsPerWave; p0 += rows_per_pass) {
        int rr = p0 + sub;
        int64_t r = row0 + rr;
        bool is_v = false;
        if (m.store) {
            int64_t t = r / (2 * m.H);
            is_v = (int)(r - t * 2 * m.H) >= m.H;
        }
        float x[8];
        load8<S>(lds + rr * row_pitch + part * 8 * EB, x);
        float den = lds_norm[rr] + 1e-10f;
        float xn[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) xn[e] = x[e] / den;
        int nb = is_v ? nvb : nkb;
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            int kb0 = (e / BLK) * BLK;  // block start inside this lane's 8 elements
            float acc = xn[kb0] * rt[e][0];
#pragma unroll
            for (int i = 1; i < BLK; ++i) acc = __builtin_fmaf(xn[kb0 + i], rt[e][i], acc);
            uint32_t idx = 0;
#pragma unroll
            for (int b = 0; b < kMaxBounds; ++b) {
                float bb = is_v ? vb[b] : kb[b];
                idx += (b < nb && bb < acc) ? 1u : 0u;
            }
            // byte e/2: even coordinate in the high nibble, odd in the low one
            word |= idx << (8 * (e >> 1) + ((e & 1) ? 0 : 4));
        }
        if (r < n_rows) {
            if (!m.store) {
                reinterpret_cast<uint32_t *>(m.packed + r * (int64_t)half)[part] = word;
            } else {
                int64_t t = r / (2 * m.H);
                int rem = (int)(r - t * 2 * m.H);
                int h = is_v ? rem - m.H : rem;
                uint8_t *base = slot_base(m, t);
                SlotLayout L(m.H, D);
                if (base != nullptr)
                    reinterpret_cast<uint32_t *>(base + (is_v ? L.v_idx : L.k_idx) + h * half)[part] = word;
            }
        }
    }
}

template <int DT, int BLK>
static int launch_compress_blk(const RowMap &m, int64_t n_rows, int D, const float *rte, const float *rto,
                               const float *kb, int nkb, const float *vb, int nvb, hipStream_t st) {
    int eb = DT == RQ_DTYPE_F32 ? 4 : 2;
    size_t lds = (size_t)kRowsPerWave * (D * eb + 16) + kRowsPerWave * sizeof(float);
    int64_t grid = (n_rows + kRowsPerWave - 1) / kRowsPerWave;
    hipLaunchKernelGGL((compress_kernel<DT, BLK>), dim3((unsigned)grid), dim3(64), lds, st, m, n_rows, D, rte, rto,
                       kb, nkb, vb, nvb);
    return check_launch("compress_kernel");
}

template <int DT>
static int launch_compress(const RowMap &m, int64_t n_rows, int D, const float *rte, const float *rto, int blk,
                           const float *kb, int nkb, const float *vb, int nvb, hipStream_t st) {
    if (n_rows == 0) return RQ_OK;
    switch (blk) {
        case 2: return launch_compress_blk<DT, 2>(m, n_rows, D, rte, rto, kb, nkb, vb, nvb, st);
        case 4: return launch_compress_blk<DT, 4>(m, n_rows, D, rte, rto, kb, nkb, vb, nvb, st);
        case 8: return launch_compress_blk<DT, 8>(m, n_rows, D, rte, rto, kb, nkb, vb, nvb, st);
    }
    set_error("rot_block %d unsupported", blk);
    return RQ_EINVAL;
}

static int dispatch_compress(int dtype, const RowMap &m, int64_t n_rows, int D, const float *rte, const float *rto,
                             int blk, const float *kb, int nkb, const float *vb, int nvb, hipStream_t st) {
    switch (dtype) {
        case RQ_DTYPE_F16: return launch_compress<RQ_DTYPE_F16>(m, n_rows, D, rte, rto, blk, kb, nkb, vb, nvb, st);
        case RQ_DTYPE_BF16: return launch_compress<RQ_DTYPE_BF16>(m, n_rows, D, rte, rto, blk, kb, nkb, vb, nvb, st);
        case RQ_DTYPE_F32: return launch_compress<RQ_DTYPE_F32>(m, n_rows, D, rte, rto, blk, kb, nkb, vb, nvb, st);
    }
    set_error("unsupported dtype %d", dtype);
    return RQ_EINVAL;
}

static int check_common(int dtype, int D, int blk, int nkb, int nvb) {
    RQ_CHECK_ARG(dtype == RQ_DTYPE_F16 || dtype == RQ_DTYPE_BF16 || dtype == RQ_DTYPE_F32, "bad dtype %d", dtype);
    RQ_CHECK_ARG(D % 16 == 0 && D >= 16 && D <= kMaxD, "head_dim %d must be a multiple of 16 in [16, %d]", D, kMaxD);
    RQ_CHECK_ARG(blk == 2 || blk == 4 || blk == 8, "rot_block %d must be 2, 4 or 8", blk);
    RQ_CHECK_ARG(nkb >= 1 && nkb <= kMaxBounds && nvb >= 1 && nvb <= kMaxBounds, "boundary count must be 1..15");
    return RQ_OK;
}

}  // namespace rq

using namespace rq;

extern "C" int rq_compress(const void *x, int32_t x_dtype, int64_t n_rows, int32_t head_dim,
                           const float *rot_t_even, const float *rot_t_odd, int32_t rot_block,
                           const float *boundaries, int32_t n_boundaries, uint8_t *packed, float *norms,
                           void *stream) {
    int rc = check_common(x_dtype, head_dim, rot_block, n_boundaries, n_boundaries);
    if (rc) return rc;
    RQ_CHECK_ARG(n_rows >= 0, "n_rows < 0");
    RQ_CHECK_ARG(n_rows == 0 || (x && packed && norms && rot_t_even && rot_t_odd && boundaries), "null pointer");
    RQ_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)packed % 4) == 0 && ((uintptr_t)norms % 4) == 0,
                 "x must be 16-byte aligned, packed/norms 4-byte aligned");
    RowMap m{};
    m.store = 0;
    m.x = x;
    m.packed = packed;
    m.norms = norms;
    m.H = 1;
    return dispatch_compress(x_dtype, m, n_rows, head_dim, rot_t_even, rot_t_odd, rot_block, boundaries,
                             n_boundaries, boundaries, n_boundaries, (hipStream_t)stream);
}

extern "C" int rq_compress_store(const void *key, const void *value, int32_t dtype, int64_t n_tokens,
                                 int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_token,
                                 int64_t v_stride_head, int32_t num_kv_heads, int32_t head_dim,
                                 const int64_t *slot_mapping, uint8_t *kv_cache, int64_t num_blocks,
                                 int32_t block_size, int64_t stride_block, int64_t stride_token,
                                 int32_t total_bytes, const float *rot_t_even, const float *rot_t_odd,
                                 int32_t rot_block, const float *k_boundaries, int32_t n_k_boundaries,
                                 const float *v_boundaries, int32_t n_v_boundaries, void *stream) {
    int rc = check_common(dtype, head_dim, rot_block, n_k_boundaries, n_v_boundaries);
    if (rc) return rc;
    RQ_CHECK_ARG(num_kv_heads >= 1 && n_tokens >= 0 && block_size >= 1 && num_blocks >= 0, "bad sizes");
    if (n_tokens == 0) return RQ_OK;
    RQ_CHECK_ARG(key && value && slot_mapping && kv_cache && rot_t_even && rot_t_odd && k_boundaries && v_boundaries,
                 "null pointer");
    SlotLayout L(num_kv_heads, head_dim);
    RQ_CHECK_ARG(total_bytes >= L.payload && total_bytes % 4 == 0, "total_bytes %d < payload %d or not 4-aligned",
                 total_bytes, L.payload);
    RQ_CHECK_ARG(stride_token >= total_bytes && stride_token % 4 == 0 && stride_block % 4 == 0,
                 "cache strides must be >= total_bytes and 4-aligned");
    RQ_CHECK_ARG(((uintptr_t)kv_cache % 4) == 0, "kv_cache must be 4-byte aligned");
    int eb = dtype == RQ_DTYPE_F32 ? 4 : 2;
    RQ_CHECK_ARG(((uintptr_t)key % 16) == 0 && ((uintptr_t)value % 16) == 0 && (k_stride_token * eb) % 16 == 0 &&
                     (k_stride_head * eb) % 16 == 0 && (v_stride_token * eb) % 16 == 0 &&
                     (v_stride_head * eb) % 16 == 0,
                 "key/value rows must be 16-byte aligned");
    RowMap m{};
    m.store = 1;
    m.key = key;
    m.value = value;
    m.k_st = k_stride_token;
    m.k_sh = k_stride_head;
    m.v_st = v_stride_token;
    m.v_sh = v_stride_head;
    m.slot_mapping = slot_mapping;
    m.cache = kv_cache;
    m.block_size = block_size;
    m.num_slots = num_blocks * block_size;
    m.stride_block = stride_block;
    m.stride_token = stride_token;
    m.total_bytes = total_bytes;
    m.H = num_kv_heads;
    int64_t n_rows = n_tokens * 2 * num_kv_heads;
    return dispatch_compress(dtype, m, n_rows, head_dim, rot_t_even, rot_t_odd, rot_block, k_boundaries,
                             n_k_boundaries, v_boundaries, n_v_boundaries, (hipStream_t)stream);
}
