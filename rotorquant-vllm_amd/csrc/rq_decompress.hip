// Decompress kernels: nibble unpack -> centroid -> x norm -> cast, in rotated
// space (no inverse rotation), bit-exact with the reference's CPU fallback
// (src/rotorquant_vllm/triton/isoquant_decompress.py:103-133): one fp32
// multiply centroid[idx] * norm, then a round-to-nearest-even cast.
//
// The paged variant replaces RQAttentionImpl._decompress_cache_paged
// (src/rotorquant_vllm/vllm/rq_backend.py:737-852).  Instead of
// torch.unique + gather + per-head stack it runs four small kernels:
//   mark    : flag[p] = 1 for every physical block p referenced by a
//             sequence's first ceil(len / block_size) table entries;
//   scan    : compact[p] = exclusive prefix sum of flag (ascending physical
//             order, i.e. the order of the reference's sorted unique);
//   expand  : each flagged block is decompressed once into out[compact[p]];
//   remap   : remapped[b][j] = flag[bt[b][j]] ? compact[bt[b][j]] : 0.
#include "rq_common.h"

namespace rq {

template <int DT>
__device__ __forceinline__ void store8(void *out, int64_t elem_off, const float (&v)[8]) {
    if constexpr (DT == RQ_DTYPE_F32) {
        float4 *p = reinterpret_cast<float4 *>(reinterpret_cast<float *>(out) + elem_off);
        p[0] = make_float4(v[0], v[1], v[2], v[3]);
        p[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = Elem<DT>::from_f32(v[2 * i]) | (Elem<DT>::from_f32(v[2 * i + 1]) << 16);
        typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
        __builtin_nontemporal_store((u32x4_t){w[0], w[1], w[2], w[3]},
                                    reinterpret_cast<u32x4_t *>(reinterpret_cast<uint16_t *>(out) + elem_off));
    }
}

// 8 values from one packed dword: byte i holds (even, odd) = (hi, lo) nibble.
__device__ __forceinline__ void unpack8(uint32_t word, const float *cb, float norm, float (&v)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t byte = (word >> (8 * i)) & 0xffu;
        v[2 * i] = opaque(cb[byte >> 4] * norm);
        v[2 * i + 1] = opaque(cb[byte & 15u] * norm);
    }
}

// One thread per packed dword (8 coordinates).
template <int DT>
__global__ __launch_bounds__(256) void decompress_kernel(const uint8_t *__restrict__ packed,
                                                         const float *__restrict__ norms, int64_t n_rows, int D,
                                                         const float *__restrict__ centroids, int n_c, void *out) {
    __shared__ float cb[16];
    if (threadIdx.x < 16) cb[threadIdx.x] = threadIdx.x < (unsigned)n_c ? centroids[threadIdx.x] : 0.f;
    __syncthreads();
    const int words = D / 8;
    const int64_t total = n_rows * words;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t r = i / words;
        int w = (int)(i - r * words);
        uint32_t word = reinterpret_cast<const uint32_t *>(packed + r * (D / 2))[w];
        float v[8];
        unpack8(word, cb, norms[r], v);
        store8<DT>(out, r * D + w * 8, v);
    }
}

__global__ void zero_i32_kernel(int32_t *p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0;
}

__global__ void mark_kernel(const int32_t *__restrict__ bt, int64_t num_seqs, int64_t max_blocks, int64_t bt_stride,
                            const int32_t *__restrict__ seq_lens, int block_size, int64_t num_blocks,
                            int32_t *__restrict__ flag) {
    int64_t b = blockIdx.y;
    int64_t nb = ((int64_t)seq_lens[b] + block_size - 1) / block_size;
    if (nb > max_blocks) nb = max_blocks;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < nb; j += (int64_t)gridDim.x * blockDim.x) {
        int32_t p = bt[b * bt_stride + j];
        if (p >= 0 && p < num_blocks) flag[p] = 1;
    }
}

// Single-workgroup exclusive scan of flag[0..n) into compact[], total into *count.
// Thread t owns a contiguous run of a multiple of 4 entries (16-byte loads and
// stores; flag and compact are 16-byte aligned), four loads in flight per step.
__global__ __launch_bounds__(1024) void scan_kernel(const int32_t *__restrict__ flag, int32_t *__restrict__ compact,
                                                     int64_t n, int32_t *count) {
    __shared__ int32_t part[1024];
    const int tid = threadIdx.x;
    const int64_t per = (((n + 1023) / 1024) + 3) & ~(int64_t)3;
    const int64_t beg = tid * per < n ? tid * per : n, end = beg + per < n ? beg + per : n;
    const int64_t nv = (end - beg) >> 2;  // whole 4-entry groups
    const int4 *f4 = reinterpret_cast<const int4 *>(flag + beg);
    int32_t s = 0;
#pragma unroll 4
    for (int64_t k = 0; k < nv; ++k) {
        const int4 x = f4[k];
        s += x.x + x.y + x.z + x.w;
    }
    for (int64_t i = beg + 4 * nv; i < end; ++i) s += flag[i];
    part[tid] = s;
    __syncthreads();
    // Hillis-Steele inclusive scan over the 1024 partial sums.
    for (int off = 1; off < 1024; off <<= 1) {
        int32_t v = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    int32_t run = part[tid] - s;
    int4 *c4 = reinterpret_cast<int4 *>(compact + beg);
#pragma unroll 4
    for (int64_t k = 0; k < nv; ++k) {
        const int4 x = f4[k];
        int4 o;
        o.x = run;
        o.y = run + x.x;
        o.z = o.y + x.y;
        o.w = o.z + x.z;
        run = o.w + x.w;
        c4[k] = o;
    }
    for (int64_t i = beg + 4 * nv; i < end; ++i) {
        compact[i] = run;
        run += flag[i];
    }
    if (tid == 1023 && count) *count = part[1023];
}

// One workgroup per physical block: decompress its block_size x H x (K, V) rows.
template <int DT>
__global__ __launch_bounds__(256) void expand_kernel(const uint8_t *__restrict__ cache, int block_size,
                                                     int64_t stride_block, int64_t stride_token, int H, int D,
                                                     const int32_t *__restrict__ flag,
                                                     const int32_t *__restrict__ compact, int64_t capacity,
                                                     const float *__restrict__ kc, int nkc,
                                                     const float *__restrict__ vc, int nvc, void *out_k,
                                                     void *out_v, int dense3) {
    __shared__ float cbk[16], cbv[16];
    const int64_t p = blockIdx.x;
    if (threadIdx.x < 16) {
        cbk[threadIdx.x] = threadIdx.x < (unsigned)nkc ? kc[threadIdx.x] : 0.f;
        cbv[threadIdx.x] = threadIdx.x < (unsigned)nvc ? vc[threadIdx.x] : 0.f;
    }
    __syncthreads();
    if (!flag[p]) return;
    const int64_t c = compact[p];
    if (c >= capacity) return;
    SlotLayout L(H, D, dense3 != 0);
    // Rows are (component, token, head); a row has D / 8 packed dwords.  The launch
    // uses a multiple of D / 8 threads, so each thread keeps one dword position w and
    // steps over rows: one division (by H) per row instead of three per dword.  The
    // rows go in batches of kBatch per thread whose index and norm loads are all issued
    // before any is used: one row at a time, every row waited out a full load latency.
    constexpr int kBatch = 16;
    const int words = D / 8;
    const int rows_per_comp = block_size * H, nrows = 2 * rows_per_comp;
    const int w = threadIdx.x % words, rstep = blockDim.x / words;
    for (int r0 = threadIdx.x / words; r0 < nrows; r0 += kBatch * rstep) {
        uint32_t word[kBatch];
        float norm[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int r = r0 + u * rstep;
            word[u] = 0u;
            norm[u] = 0.f;
            if (r < nrows) {
                const int comp = r >= rows_per_comp ? 1 : 0;  // 0 = K, 1 = V
                const int rr = r - comp * rows_per_comp;
                const int tok = (int)((uint32_t)rr / (uint32_t)H), h = rr - tok * H;
                const uint8_t *slot = cache + p * stride_block + (int64_t)tok * stride_token;
                word[u] = idx_dword(slot + (comp ? L.v_idx : L.k_idx) + h * L.ib, w, dense3 != 0);
                norm[u] = *reinterpret_cast<const float *>(slot + (comp ? L.v_norm : L.k_norm) + 4 * h);
            }
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int r = r0 + u * rstep;
            if (r < nrows) {
                const int comp = r >= rows_per_comp ? 1 : 0;
                const int rr = r - comp * rows_per_comp;
                float v[8];
                unpack8(word[u], comp ? cbv : cbk, norm[u], v);
                const int64_t off = (c * rows_per_comp + rr) * (int64_t)D + w * 8;  // row (c, tok, h) of the output
                store8<DT>(comp ? out_v : out_k, off, v);
            }
        }
    }
}

__global__ void remap_kernel(const int32_t *__restrict__ bt, int64_t num_seqs, int64_t max_blocks, int64_t bt_stride,
                             int64_t num_blocks, const int32_t *__restrict__ flag,
                             const int32_t *__restrict__ compact, int32_t *__restrict__ out) {
    int64_t total = num_seqs * max_blocks;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t b = i / max_blocks, j = i - b * max_blocks;
        int32_t p = bt[b * bt_stride + j];
        out[i] = (p >= 0 && p < num_blocks && flag[p]) ? compact[p] : 0;
    }
}

static int grid_for(int64_t n, int threads) {
    int64_t g = (n + threads - 1) / threads;
    if (g > 65535 * 4) g = 65535 * 4;
    return (int)(g < 1 ? 1 : g);
}

}  // namespace rq

using namespace rq;

extern "C" int rq_decompress(const uint8_t *packed, const float *norms, int64_t n_rows, int32_t head_dim,
                             const float *centroids, int32_t n_centroids, void *out, int32_t out_dtype,
                             void *stream) {
    RQ_CHECK_ARG(head_dim % 16 == 0 && head_dim >= 16, "head_dim %d must be a multiple of 16", head_dim);
    RQ_CHECK_ARG(n_centroids >= 1 && n_centroids <= 16, "n_centroids %d must be 1..16", n_centroids);
    RQ_CHECK_ARG(n_rows >= 0, "n_rows < 0");
    if (n_rows == 0) return RQ_OK;
    RQ_CHECK_ARG(packed && norms && centroids && out, "null pointer");
    RQ_CHECK_ARG(((uintptr_t)packed % 4) == 0 && ((uintptr_t)out % 16) == 0, "alignment: packed 4 B, out 16 B");
    hipStream_t st = (hipStream_t)stream;
    int grid = grid_for(n_rows * (head_dim / 8), 256);
    switch (out_dtype) {
        case RQ_DTYPE_F16:
            hipLaunchKernelGGL(decompress_kernel<RQ_DTYPE_F16>, dim3(grid), dim3(256), 0, st, packed, norms, n_rows,
                               head_dim, centroids, n_centroids, out);
            break;
        case RQ_DTYPE_BF16:
            hipLaunchKernelGGL(decompress_kernel<RQ_DTYPE_BF16>, dim3(grid), dim3(256), 0, st, packed, norms, n_rows,
                               head_dim, centroids, n_centroids, out);
            break;
        case RQ_DTYPE_F32:
            hipLaunchKernelGGL(decompress_kernel<RQ_DTYPE_F32>, dim3(grid), dim3(256), 0, st, packed, norms, n_rows,
                               head_dim, centroids, n_centroids, out);
            break;
        default: set_error("bad out_dtype %d", out_dtype); return RQ_EINVAL;
    }
    return check_launch("decompress_kernel");
}

extern "C" int64_t rq_paged_decompress_workspace_bytes(int64_t num_blocks) {
    return 2 * num_blocks * (int64_t)sizeof(int32_t) + 256;
}

extern "C" int rq_paged_decompress(const uint8_t *kv_cache, int64_t num_blocks, int32_t block_size,
                                   int64_t stride_block, int64_t stride_token, int32_t num_kv_heads,
                                   int32_t head_dim, int32_t index_layout, const int32_t *block_table,
                                   int64_t num_seqs,
                                   int64_t max_blocks, int64_t bt_stride_seq, const int32_t *seq_lens,
                                   const float *k_centroids, int32_t n_k_centroids, const float *v_centroids,
                                   int32_t n_v_centroids, void *out_k, void *out_v, int32_t out_dtype,
                                   int64_t capacity_blocks, int32_t *remapped_block_table, int32_t *num_unique,
                                   void *workspace, int64_t workspace_bytes, void *stream) {
    RQ_CHECK_ARG(head_dim % 16 == 0 && head_dim >= 16 && head_dim <= 8192, "head_dim %d must be a multiple of 16 in 16..8192", head_dim);
    RQ_CHECK_ARG(num_kv_heads >= 1 && block_size >= 1 && num_blocks >= 0 && num_seqs >= 0 && max_blocks >= 0,
                 "bad sizes");
    RQ_CHECK_ARG(n_k_centroids >= 1 && n_k_centroids <= 16 && n_v_centroids >= 1 && n_v_centroids <= 16,
                 "centroid counts must be 1..16");
    const int lrc = check_index_layout(index_layout, head_dim, n_k_centroids, n_v_centroids);
    if (lrc) return lrc;
    RQ_CHECK_ARG(out_dtype == RQ_DTYPE_F16 || out_dtype == RQ_DTYPE_BF16 || out_dtype == RQ_DTYPE_F32,
                 "bad out_dtype %d", out_dtype);
    RQ_CHECK_SPACE(workspace_bytes >= rq_paged_decompress_workspace_bytes(num_blocks), "workspace too small");
    RQ_CHECK_ARG(((uintptr_t)workspace % 16) == 0, "workspace must be 16-byte aligned");
    RQ_CHECK_ARG(stride_token % 4 == 0 && stride_block % 4 == 0 && ((uintptr_t)kv_cache % 4) == 0,
                 "cache must be 4-byte aligned");
    RQ_CHECK_ARG(((uintptr_t)out_k % 16) == 0 && ((uintptr_t)out_v % 16) == 0, "outputs must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    int32_t *flag = reinterpret_cast<int32_t *>(workspace);
    int32_t *compact = flag + ((num_blocks + 3) & ~(int64_t)3);  // 16-byte aligned (within the 256-byte slack)
    if (num_blocks > 0) {
        hipLaunchKernelGGL(zero_i32_kernel, dim3(grid_for(num_blocks, 256)), dim3(256), 0, st, flag, num_blocks);
        if (num_seqs > 0 && max_blocks > 0)
            hipLaunchKernelGGL(mark_kernel, dim3(grid_for(max_blocks, 256), (unsigned)num_seqs), dim3(256), 0, st,
                               block_table, num_seqs, max_blocks, bt_stride_seq, seq_lens, block_size, num_blocks,
                               flag);
        hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, st, flag, compact, num_blocks, num_unique);
        if (capacity_blocks > 0) {
            const int wpr = head_dim / 8;  // packed dwords per row; the block is a multiple of it
            const int ethreads = wpr >= 256 ? wpr : (256 / wpr) * wpr;
            switch (out_dtype) {
#define RQ_EXPAND(DT)                                                                                              \
    hipLaunchKernelGGL(expand_kernel<DT>, dim3((unsigned)num_blocks), dim3(ethreads), 0, st, kv_cache, block_size, \
                       stride_block, stride_token, num_kv_heads, head_dim, flag, compact, capacity_blocks,         \
                       k_centroids, n_k_centroids, v_centroids, n_v_centroids, out_k, out_v,                      \
                       index_layout == RQ_INDEX_DENSE3)
                case RQ_DTYPE_F16: RQ_EXPAND(RQ_DTYPE_F16); break;
                case RQ_DTYPE_BF16: RQ_EXPAND(RQ_DTYPE_BF16); break;
                default: RQ_EXPAND(RQ_DTYPE_F32); break;
#undef RQ_EXPAND
            }
        }
    } else if (num_unique) {
        hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(64), 0, st, num_unique, 1);
    }
    if (remapped_block_table && num_seqs * max_blocks > 0)
        hipLaunchKernelGGL(remap_kernel, dim3(grid_for(num_seqs * max_blocks, 256)), dim3(256), 0, st, block_table,
                           num_seqs, max_blocks, bt_stride_seq, num_blocks, flag, compact, remapped_block_table);
    return check_launch("paged_decompress");
}
