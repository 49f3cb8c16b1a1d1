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
// How the kernel meets that contract cheaply:
//   * divide: per row, y_hi = RN(1/d) and y_lo = RN(RN(1 - d*y_hi) * y_hi), so
//     y_hi + y_lo is 1/d to about 2^-46.  Per element, q0 = fma(x, y_hi, x*y_lo)
//     is then within one ulp of x/d, r = fma(-q0, d, x) is exact and
//     fma(r, y_hi, q0) = RN(x/d) by Markstein's theorem (y_hi correctly rounded,
//     q0 within one ulp), provided nothing underflows; rows or elements outside
//     the guarded range (d > 2^40, or 0 < |x| < 2^-60) use the plain division.
//     fp16 elements enter these fmas directly through v_fma_mix_f32.
//   * index : a 256-cell table over a monotone map cell(v) = u8(fma(v, s, c))
//     (one saturating convert) replaces the 15 comparisons.  Because cell() is monotone, every boundary
//     in a lower cell than v is < v and every boundary in a higher cell is > v;
//     when each cell holds at most one boundary (checked per workgroup), the
//     count is table[cell].n + (table[cell].b < v).  Boundary sets that fail the
//     check (NaNs, unsorted, too close together) take the 15-comparison count.
//
// Work split: rows (one row = one (token, head) of K or V) go in groups of 64
// to persistent workgroups of four waves, one group after another.  While a
// group is processed, the next group's row addresses are resolved and its rows
// are already loading into registers.  A group's rows are staged through LDS
// with coalesced 16-byte loads; four lanes per row reduce the norm's partial
// sums; D/8 lanes per row then produce 8 indices each (one packed dword).
#include "rq_common.h"

namespace rq {

constexpr int kRows = 64;        // rows per workgroup
constexpr int kThreads = 256;    // four waves
constexpr int kMaxBounds = 15;
constexpr int kMaxD = 256;
constexpr int kCells = 256;      // bucketize lookup cells per boundary set (the u8 convert's range)

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
    int32_t pad_vec;    // slot padding can be cleared with 16-byte stores
    int32_t dense3;     // store mode: dense 3-bit index layout
};

// Per-row addresses, resolved once per workgroup.
struct RowRef {
    const uint8_t *src;  // first element (nullptr: row past the end)
    uint8_t *idx_dst;    // packed indices (nullptr: row past the end or slot skipped)
    float *norm_dst;
    int32_t is_v, pad;
};

// LDS map of one workgroup (bytes).  Row addresses and padding lists are
// double-buffered: the next group's are resolved while the current one is used.
constexpr int kOffRefs = 0;                                  // RowRef[2][kRows]
constexpr int kOffTbl = kOffRefs + 2 * kRows * 32;           // float2[2][kCells]: {boundary, count}
constexpr int kOffBnd = kOffTbl + 2 * kCells * 8;            // float[2][16]
constexpr int kOffCell = kOffBnd + 2 * 16 * 4;               // int[2][16]
constexpr int kOffPad = kOffCell + 2 * 16 * 4;               // uint8_t *[2][kRows / 2]
constexpr int kOffMisc = kOffPad + 2 * (kRows / 2) * 8;      // int: pad count [2], table flag
constexpr int kOffRowp = kOffMisc + 16;                      // float4[kRows]: d, y_hi, y_lo, fast
constexpr int kOffRows = kOffRowp + kRows * 16;
static_assert(sizeof(RowRef) == 32, "RowRef layout");

// Global-memory view of a pointer that was read back from LDS (the compiler
// cannot infer its address space; flat accesses would also count against the
// LDS wait counter).
// (The host pass of this single-source file only parses device code, so there
// the view is the plain pointer.)
#if defined(__HIP_DEVICE_COMPILE__)
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T *gbl(T *p) {
    return (__attribute__((address_space(1))) T *)p;
}
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T *gbl(const T *p) {
    return (const __attribute__((address_space(1))) T *)p;
}
#else
template <typename T>
__device__ __forceinline__ T *gbl(T *p) { return p; }
#endif

// Byte address of a token's slot given its slot id (nullptr when the slot is < 0
// or past the cache).
__device__ __forceinline__ uint8_t *slot_base(const RowMap &m, int64_t s) {
    if (s < 0 || s >= m.num_slots) return nullptr;
    int64_t blk, off;
    if (m.num_slots <= 0x7fffffff) {
        uint32_t b = (uint32_t)s / (uint32_t)m.block_size;
        blk = b;
        off = (int64_t)((uint32_t)s - b * (uint32_t)m.block_size);
    } else {
        blk = s / m.block_size;
        off = s - blk * m.block_size;
    }
    return m.cache + blk * m.stride_block + off * m.stride_token;
}

// Monotone (non-decreasing) map of a value to a lookup cell: v_cvt_pk_u8_f32 rounds
// to an integer and saturates to [0, 255] (NaN -> 0) in one instruction, so the map
// is defined for every input and needs no clamp.
__device__ __forceinline__ int cell_of(float v, float s, float c) {
    const float t = __builtin_fmaf(v, s, c);
    uint32_t i;
    asm("v_cvt_pk_u8_f32 %0, %1, 0, 0" : "=v"(i) : "v"(t));
    return (int)i;
}

// Mixed-precision fused multiply-adds (v_fma_mix_f32): the f16 operand is the
// low (HI = 0) or high (HI = 1) half of a dword and enters the fma exactly.
template <int HI>
__device__ __forceinline__ float mix_fma(uint32_t w, float b, float c) {  // x * b + c
    float d;
    if constexpr (HI) asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(w), "v"(b), "v"(c));
    else asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(w), "v"(b), "v"(c));
    return d;
}
template <int HI>
__device__ __forceinline__ float mix_fnma(float a, float b, uint32_t w) {  // -a * b + x
    float d;
    if constexpr (HI) asm("v_fma_mix_f32 %0, -%1, %2, %3 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "=v"(d) : "v"(a), "v"(b), "v"(w));
    else asm("v_fma_mix_f32 %0, -%1, %2, %3 op_sel:[0,0,0] op_sel_hi:[0,0,1]" : "=v"(d) : "v"(a), "v"(b), "v"(w));
    return d;
}
template <int HI>
__device__ __forceinline__ float mix_sq(uint32_t w, float s) {  // x * x + s
    float d;
    if constexpr (HI) asm("v_fma_mix_f32 %0, %1, %1, %2 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "=v"(d) : "v"(w), "v"(s));
    else asm("v_fma_mix_f32 %0, %1, %1, %2 op_sel:[0,0,0] op_sel_hi:[1,1,0]" : "=v"(d) : "v"(w), "v"(s));
    return d;
}

// x / d for the guarded range, from y_hi = RN(1/d) and y_lo = RN(RN(1 - d*y_hi) * y_hi)
// (y_hi + y_lo = 1/d to about 2^-46): q0 = fma(x, y_hi, x*y_lo) is within one ulp of
// x/d, r = fma(-q0, d, x) is exact, and fma(r, y_hi, q0) = RN(x/d) (Markstein).
__device__ __forceinline__ float div_dd(float x, float d, float yh, float yl) {
    const float q0 = __builtin_fmaf(x, yh, x * yl);
    const float r = __builtin_fmaf(-q0, d, x);
    return __builtin_fmaf(r, yh, q0);
}
template <int HI>
__device__ __forceinline__ float div_dd_f16(uint32_t w, float d, float yh, float yl) {
    const float q0 = mix_fma<HI>(w, yh, mix_fma<HI>(w, yl, 0.f));
    const float r = mix_fnma<HI>(q0, d, w);
    return __builtin_fmaf(r, yh, q0);
}

template <int DT> struct Src;
template <> struct Src<RQ_DTYPE_F16> : Elem<RQ_DTYPE_F16> { static constexpr int bytes = 2; };
template <> struct Src<RQ_DTYPE_BF16> : Elem<RQ_DTYPE_BF16> { static constexpr int bytes = 2; };
template <> struct Src<RQ_DTYPE_F32> { static constexpr int bytes = 4; };

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

template <typename T>
__device__ __forceinline__ void load2(const uint8_t *lds, float &a, float &b) {
    if constexpr (T::bytes == 2) {
        uint32_t w = *reinterpret_cast<const uint32_t *>(lds);
        a = T::to_f32(w & 0xffffu);
        b = T::to_f32(w >> 16);
    } else {
        float2 v = *reinterpret_cast<const float2 *>(lds);
        a = v.x;
        b = v.y;
    }
}

// Scale and offset of the cell map for one boundary set: cell(b_0) = 0 and
// cell(b_last) = kCells - 1 up to rounding; s = 0 when the span is empty or not finite.
__device__ __forceinline__ void cell_params(const float *__restrict__ bnd, int nb, float &s, float &c) {
    const float lo = bnd[0], span = bnd[nb - 1] - lo;
    s = (span > 0.f && span < 3.0e38f) ? (float)(kCells - 1) / span : 0.f;
    if (!(s < 1.0e30f)) s = 0.f;
    c = -lo * s;
    if (!(fabsf(c) < 1.0e30f)) { s = 0.f; c = 0.f; }
}

// Position of a group of kRows rows in store mode: first row, its token and the
// row's index inside that token (rows of a token: K heads, then V heads).
struct Cursor {
    int64_t row0, tok0;
    int rem0;
};

// Four resident waves per SIMD (at most 128 VGPRs) measured fastest for rotation
// blocks up to 4; 8x8 blocks keep their registers.
constexpr int compress_waves_per_eu(int blk) { return blk <= 4 ? 4 : 1; }

// DC: head_dim fixed at compile time (128: every loop has a constant trip count), 0 = runtime D_in.
template <int DT, int BLK, int DC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(compress_waves_per_eu(BLK)))) void compress_kernel(RowMap m, int64_t n_rows, int D_in,
                                                            const float *__restrict__ rt_even,
                                                            const float *__restrict__ rt_odd,
                                                            const float *__restrict__ kbnd, int nkb,
                                                            const float *__restrict__ vbnd, int nvb) {
    using S = Src<DT>;
    constexpr int EB = S::bytes;
    const int D = DC > 0 ? DC : D_in;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int row_bytes = D * EB;
    const int pitch = row_bytes + 16;  // +16 B keeps the per-row reads bank-conflict free
    const int half = D / 2;
    const int two_h = 2 * m.H;
    const int64_t n_groups = (n_rows + kRows - 1) / kRows;
    const int64_t gstride = gridDim.x;

    extern __shared__ __align__(16) uint8_t lds[];
    RowRef *refs_all = reinterpret_cast<RowRef *>(lds + kOffRefs);
    float2 *tbl = reinterpret_cast<float2 *>(lds + kOffTbl);
    float *bnd = reinterpret_cast<float *>(lds + kOffBnd);
    int *cells = reinterpret_cast<int *>(lds + kOffCell);
    uint8_t **pads_all = reinterpret_cast<uint8_t **>(lds + kOffPad);
    int *misc = reinterpret_cast<int *>(lds + kOffMisc);
    float4 *rowp = reinterpret_cast<float4 *>(lds + kOffRowp);
    uint8_t *rows = lds + kOffRows;

    // Quantize-step lane roles and this lane's R^T entries (loaded first).
    const int lpr = D / 8;           // lanes per row
    const int rpp = kThreads / lpr;  // rows per pass
    const int part = tid % lpr;
    const int sub = tid / lpr;
    float rt[8][BLK];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int j = part * 8 + e;
        const int k0 = (j / BLK) * BLK;
        const float *col = (j & 1) ? rt_odd : rt_even;
#pragma unroll
        for (int i = 0; i < BLK; ++i) rt[e][i] = col[(int64_t)(k0 + i) * half + (j >> 1)];
    }
    float sk, ck, sv, cv;
    cell_params(kbnd, nkb, sk, ck);
    cell_params(vbnd, nvb, sv, cv);

    // Staging roles: 16-byte piece my_part of rows my_row + u * rpi.
    const int C = row_bytes / 16;
    const int rpi = kThreads / C;
    const int my_part = tid % C, my_row = tid / C;
    const int n_it = (kRows + rpi - 1) / rpi;

    // Store-mode cursor over groups g, g + gstride, ... (wave 0 walks it).
    Cursor cur{0, 0, 0};
    int64_t step_tok = 0;
    int step_rem = 0;
    if (m.store) {
        cur.row0 = (int64_t)blockIdx.x * kRows;
        cur.tok0 = cur.row0 / two_h;
        cur.rem0 = (int)(cur.row0 - cur.tok0 * two_h);
        const int64_t step = gstride * kRows;
        step_tok = step / two_h;
        step_rem = (int)(step - step_tok * two_h);
    }
    auto advance = [&](Cursor c) {
        c.row0 += gstride * kRows;
        c.tok0 += step_tok;
        c.rem0 += step_rem;
        if (c.rem0 >= two_h) {
            c.rem0 -= two_h;
            c.tok0 += 1;
        }
        return c;
    };
    // Slot id of the token of this lane's row in the group at c (store mode, wave 0).
    auto slot_id = [&](const Cursor &c) -> int64_t {
        const int local = c.rem0 + lane;
        const int j = local / two_h;
        const int64_t t = c.tok0 + j;
        if (c.row0 + lane >= n_rows) return -1;
        return m.slot_mapping[t];
    };
    // Resolve the group's row addresses into buffer b (wave 0).
    auto build_refs = [&](const Cursor &c, int64_t g, int b, int64_t sid) {
        const int64_t r = g * kRows + lane;
        RowRef ref{nullptr, nullptr, nullptr, 0, 0};
        bool first = false;
        int pad_j = 0;
        uint8_t *base = nullptr;
        if (r < n_rows) {
            if (!m.store) {
                ref.src = reinterpret_cast<const uint8_t *>(m.x) + r * (int64_t)row_bytes;
                ref.idx_dst = m.packed + r * (int64_t)half;
                ref.norm_dst = m.norms + r;
            } else {
                const int local = c.rem0 + lane;
                const int j = local / two_h;
                const int rem = local - j * two_h;
                const int is_v = rem >= m.H;
                const int h = rem - is_v * m.H;
                const int64_t t = c.tok0 + j;
                const int64_t off =
                    is_v ? t * m.v_st + (int64_t)h * m.v_sh : t * m.k_st + (int64_t)h * m.k_sh;
                ref.src = reinterpret_cast<const uint8_t *>(is_v ? m.value : m.key) + off * EB;
                base = slot_base(m, sid);
                if (base != nullptr) {
                    const SlotLayout L(m.H, D, m.dense3 != 0);
                    ref.idx_dst = base + (is_v ? L.v_idx : L.k_idx) + h * L.ib;
                    ref.norm_dst = reinterpret_cast<float *>(base + (is_v ? L.v_norm : L.k_norm) + 4 * h);
                }
                ref.is_v = is_v;
                first = rem == 0;
                pad_j = j - (c.rem0 != 0);
            }
        }
        refs_all[b * kRows + lane] = ref;
        if (m.store) {
            if (first) pads_all[b * (kRows / 2) + pad_j] = base;
            const int npad = __popcll(__ballot(first));
            if (lane == 0) misc[b] = npad;
        }
    };
    // Batch 0 of a group's rows into registers (the rest, if any, is loaded in place).
    auto load_batch0 = [&](int b, uint4 (&v)[4]) {
        const RowRef *refs = refs_all + b * kRows;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int rr = my_row + u * rpi;
            v[u] = make_uint4(0, 0, 0, 0);
            if (my_row < rpi && u < n_it && rr < kRows) {
                const uint8_t *src = refs[rr].src;
                if (src != nullptr) v[u] = *gbl(reinterpret_cast<const uint4 *>(src + my_part * 16));
            }
        }
    };

    int64_t g = blockIdx.x;
    int64_t sid_next = -1;
    // ---- prologue: first group's addresses; boundary cells -----------------
    if (wave == 0) {
        const int64_t sid = m.store ? slot_id(cur) : -1;
        if (m.store && g + gstride < n_groups) sid_next = slot_id(advance(cur));
        build_refs(cur, g, 0, sid);
    } else if (wave == 1) {
        // lanes 0-15: K boundaries, lanes 32-47: V boundaries
        const int kind = lane >> 5, i = lane & 31;
        const int nb = kind ? nvb : nkb;
        const float *src = kind ? vbnd : kbnd;
        const float s = kind ? sv : sk, c = kind ? cv : ck;
        float b = __builtin_inff();
        int cl = kCells;
        if (i < nb) {
            b = src[i];
            cl = cell_of(b, s, c);
        }
        if (i < 16) {
            bnd[kind * 16 + i] = b;
            cells[kind * 16 + i] = cl;
        }
        // cells strictly increasing and no NaN boundary -> at most one boundary per cell
        const int next = __shfl_down(cl, 1);
        const bool bad = i < nb && (b != b || (i + 1 < nb && !(cl < next)));
        const bool all_ok = __ballot(bad) == 0ull;  // whole-wave vote, taken before lane 0 stores it
        if (lane == 0) misc[2] = all_ok;
    }
    __syncthreads();
    uint4 v[4];
    load_batch0(0, v);
    for (int e = tid; e < 2 * kCells; e += kThreads) {
        // table entry {boundary, count} of cell c for both sets
        const int kind = e / kCells, c = e % kCells;
        const int nb = kind ? nvb : nkb;
        int n = 0;
        for (int i = 0; i < nb; ++i) n += cells[kind * 16 + i] < c;
        tbl[e] = make_float2(bnd[kind * 16 + n], __int_as_float(n));
    }

    for (int buf = 0;; buf ^= 1) {
        const RowRef *refs = refs_all + buf * kRows;
        const int64_t gn = g + gstride;
        const bool has_next = gn < n_groups;
        // ---- (a) rows of g into LDS; slot padding; next group's addresses ----
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int rr = my_row + u * rpi;
            if (my_row < rpi && u < n_it && rr < kRows)
                *reinterpret_cast<uint4 *>(rows + rr * pitch + my_part * 16) = v[u];
        }
        for (int u = 4; u < n_it; ++u) {
            const int rr = my_row + u * rpi;
            if (my_row < rpi && rr < kRows) {
                const uint8_t *src = refs[rr].src;
                uint4 w = make_uint4(0, 0, 0, 0);
                if (src != nullptr) w = *gbl(reinterpret_cast<const uint4 *>(src + my_part * 16));
                *reinterpret_cast<uint4 *>(rows + rr * pitch + my_part * 16) = w;
            }
        }
        if (m.store) {
            const int pay = SlotLayout(m.H, D, m.dense3 != 0).payload;
            const int npad = misc[buf];
            uint8_t *const *pads = pads_all + buf * (kRows / 2);
            if (m.pad_vec) {
                const int units = (m.total_bytes - pay) / 16;
                for (int i = tid; i < npad * units; i += kThreads) {
                    const int j = i / units;
                    uint8_t *base = pads[j];
                    if (base != nullptr)
                        gbl(reinterpret_cast<uint4 *>(base + pay))[i - j * units] = make_uint4(0, 0, 0, 0);
                }
            } else {
                const int units = (m.total_bytes - pay) / 4;
                for (int i = tid; i < npad * units; i += kThreads) {
                    const int j = i / units;
                    uint8_t *base = pads[j];
                    if (base != nullptr) gbl(reinterpret_cast<uint32_t *>(base + pay))[i - j * units] = 0u;
                }
            }
        }
        if (wave == 0 && has_next) {
            const Cursor cn = m.store ? advance(cur) : cur;
            const int64_t sid = sid_next;
            if (m.store && gn + gstride < n_groups) sid_next = slot_id(advance(cn));
            build_refs(cn, gn, buf ^ 1, sid);
            cur = cn;
        }
        __syncthreads();
        // ---- (b) next group's rows in flight while this one is processed -----
        if (has_next) load_batch0(buf ^ 1, v);

        // ---- (c) norms, four lanes per row ------------------------------------
        // lane q of a row accumulates s_{2q} and s_{2q+1}; lane 0 adds s_0..s_7 in order
        // and prepares the row's divisor d = n + 1e-10 and its split reciprocal.
        {
            const int rr = tid >> 2, q = tid & 3;
            const uint8_t *rowq = rows + rr * pitch + 2 * q * EB;
            float s0 = 0.f, s1 = 0.f;
            for (int k = 0; k < D / 8; ++k) {
                if constexpr (DT == RQ_DTYPE_F16) {
                    const uint32_t w = *reinterpret_cast<const uint32_t *>(rowq + k * 8 * EB);
                    s0 = mix_sq<0>(w, s0);
                    s1 = mix_sq<1>(w, s1);
                } else {
                    float a, b;
                    load2<S>(rowq + k * 8 * EB, a, b);
                    s0 = __builtin_fmaf(a, a, s0);
                    s1 = __builtin_fmaf(b, b, s1);
                }
            }
            const float s2 = __shfl_down(s0, 1), s3 = __shfl_down(s1, 1);
            const float s4 = __shfl_down(s0, 2), s5 = __shfl_down(s1, 2);
            const float s6 = __shfl_down(s0, 3), s7 = __shfl_down(s1, 3);
            if (q == 0) {
                float sum = s0 + s1;
                sum = sum + s2;
                sum = sum + s3;
                sum = sum + s4;
                sum = sum + s5;
                sum = sum + s6;
                sum = sum + s7;
                const float n = __builtin_sqrtf(sum);
                const float d = n + 1e-10f;
                const float yh = 1.0f / d;
                const float yl = __builtin_fmaf(-d, yh, 1.0f) * yh;
                rowp[rr] = make_float4(d, yh, yl, d <= 0x1p40f ? 1.f : 0.f);
                float *dst = refs[rr].norm_dst;
                if (dst != nullptr) *gbl(dst) = n;
            }
        }
        __syncthreads();

        // ---- (d) D/8 lanes per row, 8 coordinates per lane ------------------
        const bool use_tbl = __builtin_amdgcn_readfirstlane(misc[2]) != 0;
        for (int rr = sub; sub < rpp && rr < kRows; rr += rpp) {
            uint32_t *dst = reinterpret_cast<uint32_t *>(refs[rr].idx_dst);
            if (dst == nullptr) continue;
            const int is_v = refs[rr].is_v;
            const float4 rp = rowp[rr];
            const float d = rp.x, yh = rp.y, yl = rp.z;
            bool fast = rp.w != 0.f;
            float xn[8];
            if constexpr (DT == RQ_DTYPE_F16) {
                // fp16 inputs are 0 or at least 2^-24 in magnitude: inside the guarded range
                const uint4 w4 = *reinterpret_cast<const uint4 *>(rows + rr * pitch + part * 16);
                const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
                if (fast) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        xn[2 * i] = div_dd_f16<0>(w[i], d, yh, yl);
                        xn[2 * i + 1] = div_dd_f16<1>(w[i], d, yh, yl);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        xn[2 * i] = S::to_f32(w[i] & 0xffffu) / d;
                        xn[2 * i + 1] = S::to_f32(w[i] >> 16) / d;
                    }
                }
            } else {
                float x[8];
                load8<S>(rows + rr * pitch + part * 8 * EB, x);
#pragma unroll
                for (int e = 0; e < 8; ++e) fast = fast && (x[e] == 0.f || fabsf(x[e]) >= 0x1p-60f);
                if (fast) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) xn[e] = div_dd(x[e], d, yh, yl);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) xn[e] = x[e] / d;
                }
            }
            float acc[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int kb0 = (e / BLK) * BLK;  // block start inside this lane's 8 elements
                float a = xn[kb0] * rt[e][0];
#pragma unroll
                for (int i = 1; i < BLK; ++i) a = __builtin_fmaf(xn[kb0 + i], rt[e][i], a);
                acc[e] = a;
            }
            uint32_t word = 0;
            if (use_tbl) {
                const float s = is_v ? sv : sk, c = is_v ? cv : ck;
                const float2 *t = tbl + is_v * kCells;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float2 ent = t[cell_of(acc[e], s, c)];
                    const uint32_t idx = (uint32_t)__float_as_int(ent.y) + (ent.x < acc[e] ? 1u : 0u);
                    // byte e/2: even coordinate in the high nibble, odd in the low one
                    word |= idx << (8 * (e >> 1) + ((e & 1) ? 0 : 4));
                }
            } else {
                const float *bb = bnd + is_v * 16;
                const int nb = is_v ? nvb : nkb;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    uint32_t idx = 0;
                    for (int b = 0; b < nb; ++b) idx += bb[b] < acc[e] ? 1u : 0u;
                    word |= idx << (8 * (e >> 1) + ((e & 1) ? 0 : 4));
                }
            }
            if (m.dense3) {
                // Lanes 4G .. 4G+3 of the row hold positions 0..3 of index group G (dims
                // 32G .. 32G+31); positions 0..2 write dwords A, B, C, topped up with
                // position 3's bits.
                const uint32_t x3 = __shfl(word, (lane & ~3) | 3);
                const uint32_t e3 = (x3 >> 4) & 0x0f0f0f0fu, o3 = x3 & 0x0f0f0f0fu;
                const int w = part & 3;
                const uint32_t own = ((word >> 4) & 0x0f0f0f0fu) | ((word & 0x0f0f0f0fu) << 3);
                const uint32_t top = w == 0 ? (e3 & 0x03030303u) << 6
                                   : w == 1 ? (o3 & 0x03030303u) << 6
                                            : (((e3 >> 2) & 0x01010101u) << 6) | (((o3 >> 2) & 0x01010101u) << 7);
                if (w < 3) gbl(dst)[3 * (part >> 2) + w] = own | top;
            } else {
                gbl(dst)[part] = word;
            }
        }
        if (!has_next) break;
        g = gn;
        __syncthreads();  // rows and this buffer's addresses are reused next
    }
}

// Resident workgroups of a compress kernel on the current device (cached).
template <int DT, int BLK, int DC>
static int compress_grid(size_t lds, int64_t n_groups) {
    static int per_cu[64] = {0};
    static size_t for_lds[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (per_cu[dev] == 0 || for_lds[dev] != lds) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void *>(&compress_kernel<DT, BLK, DC>),
                                                         kThreads, lds) != hipSuccess || nb <= 0)
            nb = 4;
        per_cu[dev] = nb;
        for_lds[dev] = lds;
    }
    const int64_t g = (int64_t)per_cu[dev] * device_cus();
    return (int)(g < n_groups ? g : n_groups);
}

template <int DT, int BLK, int DC>
static int launch_compress_dc(const RowMap &m, int64_t n_rows, int D, const float *rte, const float *rto,
                              const float *kb, int nkb, const float *vb, int nvb, hipStream_t st) {
    int eb = DT == RQ_DTYPE_F32 ? 4 : 2;
    size_t lds = (size_t)kOffRows + (size_t)kRows * (D * eb + 16);
    const int grid = compress_grid<DT, BLK, DC>(lds, (n_rows + kRows - 1) / kRows);
    hipLaunchKernelGGL((compress_kernel<DT, BLK, DC>), dim3((unsigned)grid), dim3(kThreads), lds, st, m, n_rows, D, rte,
                       rto, kb, nkb, vb, nvb);
    return check_launch("compress_kernel");
}

template <int DT, int BLK>
static int launch_compress_blk(const RowMap &m, int64_t n_rows, int D, const float *rte, const float *rto,
                               const float *kb, int nkb, const float *vb, int nvb, hipStream_t st) {
    if (D == 128) return launch_compress_dc<DT, BLK, 128>(m, n_rows, D, rte, rto, kb, nkb, vb, nvb, st);
    return launch_compress_dc<DT, BLK, 0>(m, n_rows, D, rte, rto, kb, nkb, vb, nvb, st);
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
                                 int32_t index_layout, const int64_t *slot_mapping, uint8_t *kv_cache, int64_t num_blocks,
                                 int32_t block_size, int64_t stride_block, int64_t stride_token,
                                 int32_t total_bytes, const float *rot_t_even, const float *rot_t_odd,
                                 int32_t rot_block, const float *k_boundaries, int32_t n_k_boundaries,
                                 const float *v_boundaries, int32_t n_v_boundaries, void *stream) {
    int rc = check_common(dtype, head_dim, rot_block, n_k_boundaries, n_v_boundaries);
    if (rc) return rc;
    RQ_CHECK_ARG(num_kv_heads >= 1 && n_tokens >= 0 && block_size >= 1 && num_blocks >= 0, "bad sizes");
    rc = check_index_layout(index_layout, head_dim, n_k_boundaries + 1, n_v_boundaries + 1);
    if (rc) return rc;
    if (n_tokens == 0) return RQ_OK;
    RQ_CHECK_ARG(key && value && slot_mapping && kv_cache && rot_t_even && rot_t_odd && k_boundaries && v_boundaries,
                 "null pointer");
    const bool dense3 = index_layout == RQ_INDEX_DENSE3;
    SlotLayout L(num_kv_heads, head_dim, dense3);
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
    m.dense3 = dense3;
    m.pad_vec = L.payload % 16 == 0 && total_bytes % 16 == 0 && stride_token % 16 == 0 && stride_block % 16 == 0 &&
                ((uintptr_t)kv_cache % 16) == 0;
    int64_t n_rows = n_tokens * 2 * num_kv_heads;
    return dispatch_compress(dtype, m, n_rows, head_dim, rot_t_even, rot_t_odd, rot_block, k_boundaries,
                             n_k_boundaries, v_boundaries, n_v_boundaries, (hipStream_t)stream);
}
