/*
 * rq_abi.h -- C ABI of the MI355X (gfx950) RotorQuant KV-cache library
 * (librq_hip.so, built from rotorquant-vllm_amd/csrc/).
 *
 * Every entry point takes plain device pointers, element or byte strides,
 * small integer enums and a hipStream_t passed as `void *`.  None of them
 * allocates device memory, synchronises the host or keeps state between calls:
 * scratch space (split-KV partials, prefill tile images, block marks) is passed
 * in by the caller, so the calls can be captured in a HIP graph.  All launches
 * go to `stream`.
 *
 * Return value: RQ_OK (0) on success; a nonzero rq_status otherwise.  The text
 * of the last error of the calling thread is available from rq_last_error().
 *
 * Packed paged-cache layout (one token slot of `total_bytes` bytes, H = KV
 * heads, D = head_dim, HALF = D / 2), identical to the reference's
 * src/rotorquant_vllm/vllm/rq_backend.py:482-490 and :626-653:
 *
 *   [0, H*HALF)              K indices, head h at h*HALF;
 *                            byte j = (idx[2j] << 4) | idx[2j+1]
 *   [H*HALF, H*(HALF+4))     K norms, fp32 little endian, head h at H*HALF + 4h
 *   [H*(HALF+4), H*(D+4))    V indices, same packing
 *   [H*(D+4), H*(D+8))       V norms
 *   [H*(D+8), total_bytes)   zero padding (total_bytes = H * next_pow2(D + 8))
 *
 * References below are file:line in tpurtell/rotorquant-vllm.
 */
#ifndef RQ_ABI_H
#define RQ_ABI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RQ_ABI_VERSION 7  /* 2: rq_int8_prefill takes max_seq_len and a workspace; 3: rq_fused_decode_noalloc;
                              4: rq_paged_attention; 5: index_layout on the entry points that touch slots;
                              6: rq_paged_prefill; 7: rq_fused_decode_timed */

enum rq_status {
    RQ_OK = 0,
    RQ_EINVAL = 1,   /* bad shape, stride, enum or pointer */
    RQ_ENOSPACE = 2, /* caller-provided workspace too small */
    RQ_ELAUNCH = 3   /* kernel launch reported an error */
};

enum rq_dtype {
    RQ_DTYPE_F16 = 0,
    RQ_DTYPE_BF16 = 1,
    RQ_DTYPE_F32 = 2
};

/*
 * Index layout of the packed cache (the `index_layout` argument of every entry
 * point that reads or writes cache slots):
 *   RQ_INDEX_NIBBLE: the reference's slot, head_dim / 2 index bytes per head,
 *     byte j = idx[2j] << 4 | idx[2j + 1] (rq_backend.py:155-188);
 *   RQ_INDEX_DENSE3: opt-in, 3-bit indices only (8-entry codebooks, head_dim a
 *     multiple of 32): 3 head_dim / 8 bytes per head, each 32 indices of dims
 *     32G .. 32G+31 in 12 bytes (dwords A, B, C; byte k of each):
 *       A[k] = i[2k]    | i[2k+1] << 3  | (i[24+2k] & 3) << 6
 *       B[k] = i[8+2k]  | i[9+2k] << 3  | (i[25+2k] & 3) << 6
 *       C[k] = i[16+2k] | i[17+2k] << 3 | (i[24+2k] >> 2) << 6 | (i[25+2k] >> 2) << 7
 *     The slot is [K idx | K norms | V idx | V norms | pad] as before, with the
 *     smaller index parts (104 payload bytes per head at head_dim 128 instead of
 *     136).  No counterpart in the reference, whose roadmap lists 3-bit storage
 *     (PKG-INFO:110).
 */
enum rq_index_layout {
    RQ_INDEX_NIBBLE = 0,
    RQ_INDEX_DENSE3 = 1
};

/* Version of this ABI (RQ_ABI_VERSION). */
int rq_abi_version(void);

/* Message of the last failed call on the calling thread ("" if none). */
const char *rq_last_error(void);

/*
 * Compress n_rows rows of head_dim elements (contiguous, dtype x_dtype) into
 * nibble-packed centroid indices (n_rows x head_dim/2 bytes) and fp32 norms.
 *
 * Replaces iso_compress / planar_compress:
 *   src/rotorquant_vllm/triton/isoquant_compress.py:104-158 (CPU path :161-190)
 *   src/rotorquant_vllm/triton/planarquant_compress.py:100-154 (CPU path :157-186)
 *
 * rot_t_even / rot_t_odd are the even and odd columns of R^T (head_dim x
 * head_dim/2, fp32, row major), as the reference passes them.  rot_block is the
 * width of R's diagonal blocks (4 for IsoQuant, 2 for PlanarQuant, head_dim for
 * a dense R): only entries inside the diagonal blocks are read.
 * boundaries: n_boundaries (1..15) sorted fp32 Lloyd-Max boundaries.
 * Index = number of boundaries strictly below the rotated coordinate (ties go
 * to the lower bucket, as torch.bucketize(right=False) in the CPU path).
 */
int rq_compress(const void *x, int32_t x_dtype, int64_t n_rows, int32_t head_dim,
                const float *rot_t_even, const float *rot_t_odd, int32_t rot_block,
                const float *boundaries, int32_t n_boundaries,
                uint8_t *packed, float *norms, void *stream);

/*
 * Fused K+V compress written straight into the paged cache slots.
 *
 * Replaces RQAttentionImpl._compress_and_store
 *   src/rotorquant_vllm/vllm/rq_backend.py:585-657
 * (two compress launches, a row buffer and an index_put scatter there).
 *
 * key / value: n_tokens x num_kv_heads x head_dim of dtype `dtype`, addressed
 * as base + t*stride_token + h*stride_head + d (strides in elements).
 * slot_mapping: n_tokens int64 flat slot ids (block * block_size + offset);
 * slots < 0 are skipped (vLLM's padding id).  kv_cache: uint8 cache with
 * num_blocks x block_size slots addressed as block*stride_block +
 * offset*stride_token (bytes); total_bytes is the slot size to fill.
 * Every slot written gets its full payload and zero padding.
 */
int rq_compress_store(const void *key, const void *value, int32_t dtype, int64_t n_tokens,
                      int64_t k_stride_token, int64_t k_stride_head,
                      int64_t v_stride_token, int64_t v_stride_head,
                      int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                      const int64_t *slot_mapping,
                      uint8_t *kv_cache, int64_t num_blocks, int32_t block_size,
                      int64_t stride_block, int64_t stride_token, int32_t total_bytes,
                      const float *rot_t_even, const float *rot_t_odd, int32_t rot_block,
                      const float *k_boundaries, int32_t n_k_boundaries,
                      const float *v_boundaries, int32_t n_v_boundaries,
                      void *stream);

/*
 * Decompress n_rows packed rows (head_dim/2 bytes each) and fp32 norms into
 * rotated-space values centroid[idx] * norm, rounded to out_dtype.
 *
 * Replaces iso_decompress / planar_decompress:
 *   src/rotorquant_vllm/triton/isoquant_decompress.py:63-100 (CPU path :103-133)
 *   src/rotorquant_vllm/triton/planarquant_decompress.py:63-101 (CPU path :104-133)
 *
 * n_centroids is 8 or 16.  Nibbles >= n_centroids read 0.0.
 */
int rq_decompress(const uint8_t *packed, const float *norms, int64_t n_rows, int32_t head_dim,
                  const float *centroids, int32_t n_centroids,
                  void *out, int32_t out_dtype, void *stream);

/*
 * Paged decompress of every physical block referenced by the first
 * ceil(seq_lens[b] / block_size) entries of each block_table row.
 *
 * Replaces RQAttentionImpl._decompress_cache_paged
 *   src/rotorquant_vllm/vllm/rq_backend.py:737-852
 * without torch.unique: referenced blocks are marked, a prefix sum gives each
 * one its compact id in ascending physical order (the order of the sorted
 * unique in the reference), and each is decompressed once.
 *
 * workspace: at least rq_paged_decompress_workspace_bytes(num_blocks) bytes, 16-byte aligned.
 * out_k / out_v: capacity_blocks x block_size x num_kv_heads x head_dim of
 * out_dtype.  remapped_block_table: num_seqs x max_blocks int32 (same shape
 * as block_table) receiving the compact ids (entries past a sequence's
 * length read 0, as remap[block_table] does in the reference).
 * num_unique (device int32, may be NULL) receives the number of referenced
 * blocks; blocks whose compact id >= capacity_blocks are not written.
 */
int64_t rq_paged_decompress_workspace_bytes(int64_t num_blocks);
int rq_paged_decompress(const uint8_t *kv_cache, int64_t num_blocks, int32_t block_size,
                        int64_t stride_block, int64_t stride_token,
                        int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                        const int32_t *block_table, int64_t num_seqs, int64_t max_blocks,
                        int64_t bt_stride_seq, const int32_t *seq_lens,
                        const float *k_centroids, int32_t n_k_centroids,
                        const float *v_centroids, int32_t n_v_centroids,
                        void *out_k, void *out_v, int32_t out_dtype, int64_t capacity_blocks,
                        int32_t *remapped_block_table, int32_t *num_unique,
                        void *workspace, int64_t workspace_bytes, void *stream);

/*
 * Fused paged decode attention straight from the packed cache: one query
 * token per sequence, GQA heads sharing each KV read, Q rotated by R^T and the
 * output rotated back by R inside the library.
 *
 * Replaces fused_paged_rq_decode
 *   src/rotorquant_vllm/triton/fused_paged_rq_decode.py:214-312
 *   (kernel :32-206; Q pre-rotation :271, post-rotation :308).
 *
 * q: num_seqs x num_q_heads x head_dim (element strides q_stride_seq,
 * q_stride_head; unit stride over head_dim), dtype F16 or BF16.
 * out: same shape and dtype, strides out_stride_seq / out_stride_head.
 * rotation: R, head_dim x head_dim fp32 row major, block diagonal with blocks
 * of rot_block (2 or 4).  head_dim must be 128; num_q_heads / num_kv_heads
 * must be an integer <= 16; n_k_centroids / n_v_centroids 8 or 16; centroids
 * and rotation 16-byte aligned.
 * max_seq_len bounds every seq_lens entry (it sizes the work and workspace).
 * workspace: at least rq_fused_decode_workspace_bytes(...) bytes (16-byte aligned) of device
 * scratch (split partials, query operands, tile descriptors); no
 * initialisation is needed and every call rewrites what it reads, so one
 * workspace serves any number of calls (calls sharing one workspace must not
 * overlap).  Three kernel launches per call (prep, decode, merge).
 */
int64_t rq_fused_decode_workspace_bytes(int64_t num_seqs, int32_t num_q_heads,
                                        int32_t head_dim, int64_t max_seq_len);
int rq_fused_decode(const void *q, int32_t dtype, int64_t num_seqs, int32_t num_q_heads,
                    int64_t q_stride_seq, int64_t q_stride_head,
                    const uint8_t *kv_cache, int64_t num_blocks, int32_t block_size,
                    int64_t stride_block, int64_t stride_token,
                    int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                    const int32_t *block_table, int64_t max_blocks, int64_t bt_stride_seq,
                    const int32_t *seq_lens, int64_t max_seq_len,
                    const float *k_centroids, int32_t n_k_centroids,
                    const float *v_centroids, int32_t n_v_centroids,
                    const float *rotation, int32_t rot_block, float sm_scale,
                    void *out, int64_t out_stride_seq, int64_t out_stride_head,
                    void *workspace, int64_t workspace_bytes, void *stream);

/*
 * rq_fused_decode that also records event_start and event_stop (hipEvent_t,
 * created by the caller, or NULL) at the start and the end of its decode
 * kernel -- the kernel that streams the cache -- rather than around the whole
 * call, so hipEventElapsedTime gives that kernel's own duration (measurement:
 * the roofline of the dominant kernel).  No counterpart in the reference.
 * Everything else, results included, is as for rq_fused_decode.
 */
int rq_fused_decode_timed(const void *q, int32_t dtype, int64_t num_seqs, int32_t num_q_heads,
                          int64_t q_stride_seq, int64_t q_stride_head,
                          const uint8_t *kv_cache, int64_t num_blocks, int32_t block_size,
                          int64_t stride_block, int64_t stride_token,
                          int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                          const int32_t *block_table, int64_t max_blocks, int64_t bt_stride_seq,
                          const int32_t *seq_lens, int64_t max_seq_len,
                          const float *k_centroids, int32_t n_k_centroids,
                          const float *v_centroids, int32_t n_v_centroids,
                          const float *rotation, int32_t rot_block, float sm_scale,
                          void *out, int64_t out_stride_seq, int64_t out_stride_head,
                          void *workspace, int64_t workspace_bytes, void *stream,
                          void *event_start, void *event_stop);

/*
 * rq_fused_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture that may not call
 * hipMalloc, tight serving loops, harnesses that forbid allocation).  No
 * counterpart in the reference, whose Triton launch allocates its scratch
 * through torch.
 *
 * The split partials, query operands and tile descriptors live in a static
 * device array of RQ_DECODE_SCRATCH_BYTES inside the library, one per GPU,
 * held until the process ends.  A call whose rq_fused_decode_workspace_bytes(
 * num_seqs, num_q_heads, head_dim, max_seq_len) exceeds it returns RQ_ENOSPACE
 * and launches nothing.  The call allocates nothing (no hipMalloc, no library
 * allocation); its first call on a device looks up that device's array.  All
 * calls on one GPU share the array: calls that overlap in time on one GPU (two
 * streams, two threads) race and must be serialised by the caller.  Nothing in
 * the array needs clearing between calls (every call rewrites what it reads).
 * Arguments and results are those of rq_fused_decode.
 */
#define RQ_DECODE_SCRATCH_BYTES (256LL << 20)
int rq_fused_decode_noalloc(const void *q, int32_t dtype, int64_t num_seqs, int32_t num_q_heads,
                            int64_t q_stride_seq, int64_t q_stride_head,
                            const uint8_t *kv_cache, int64_t num_blocks, int32_t block_size,
                            int64_t stride_block, int64_t stride_token,
                            int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                            const int32_t *block_table, int64_t max_blocks, int64_t bt_stride_seq,
                            const int32_t *seq_lens, int64_t max_seq_len,
                            const float *k_centroids, int32_t n_k_centroids,
                            const float *v_centroids, int32_t n_v_centroids,
                            const float *rotation, int32_t rot_block, float sm_scale,
                            void *out, int64_t out_stride_seq, int64_t out_stride_head,
                            void *stream);

/*
 * Causal prefill attention over the packed cache on int8 MFMA (Q K^T and P V),
 * for any number of sequences in one launch.  Query token i of sequence b sits
 * at position seq_lens[b] - q_len_b + i, where q_len_b = cu_seqlens_q[b+1] -
 * cu_seqlens_q[b]; it attends to cache positions <= its own.
 *
 * Replaces fused_paged_rq_int8_prefill
 *   src/rotorquant_vllm/triton/fused_paged_rq_int8_prefill.py:247-363
 *   (kernel :43-239).  The reference accepts one sequence and places query i
 *   at position i; both agree when q_len == seq_len.
 *
 * q / out: total_q x num_q_heads x head_dim, strides as for rq_fused_decode
 * (q rows and the rotation 16-byte aligned).  max_q_len bounds every q_len_b; max_seq_len bounds every seq_lens[b] (keys
 * past it are not read).  workspace: rq_int8_prefill_workspace_bytes() bytes,
 * 16-byte aligned, no initialisation needed (two launches: a pack kernel
 * decodes the cache's K/V into int8 tile images there, the attention kernel
 * streams them).  Other arguments as for rq_fused_decode.
 */
int rq_int8_prefill(const void *q, int32_t dtype, int64_t total_q, int32_t num_q_heads,
                    int64_t q_stride_tok, int64_t q_stride_head,
                    const int32_t *cu_seqlens_q, int64_t num_seqs, int64_t max_q_len,
                    const uint8_t *kv_cache, int64_t num_blocks, int32_t block_size,
                    int64_t stride_block, int64_t stride_token,
                    int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                    const int32_t *block_table, int64_t max_blocks, int64_t bt_stride_seq,
                    const int32_t *seq_lens, int64_t max_seq_len,
                    const float *k_centroids, int32_t n_k_centroids,
                    const float *v_centroids, int32_t n_v_centroids,
                    const float *rotation, int32_t rot_block, float sm_scale,
                    void *out, int64_t out_stride_tok, int64_t out_stride_head,
                    void *workspace, int64_t workspace_bytes,
                    void *stream);

/* Workspace bytes rq_int8_prefill needs: one int8 tile image (33 KB)
 * per 64 keys of max_seq_len, per sequence and kv head.  No counterpart in the
 * reference, which decodes K/V inside its attention kernel. */
int64_t rq_int8_prefill_workspace_bytes(int64_t num_seqs, int32_t num_kv_heads, int64_t max_seq_len);

/*
 * Attention of new query tokens over the packed cache with K and V dequantized
 * to the q dtype inside the kernel: the backend's non-fused path in one launch,
 * with no workspace and no decompressed copy of the cache.
 *
 * Replaces, in RQAttentionImpl.forward's non-fused path
 *   src/rotorquant_vllm/vllm/rq_backend.py:937-1036:
 *   q pre-rotation (:939-941, :981), _decompress_cache_paged (:737-852) to the
 *   q dtype, vLLM's flash_attn_varlen_func over those pages (:996-1030) and the
 *   back-rotation out = out_rot R (:1032-1034).
 * K, V = dtype(centroid * norm) (the values rq_decompress writes); S = q_rot K^T
 * with exact 16-bit products and fp32 sums; softmax in fp32; out_rot rounded to
 * the q dtype before the back-rotation.  Query i of sequence b sits at position
 * seq_lens[b] - q_len_b + i; causal != 0: it attends to cache positions <= its
 * own (flash attention's bottom-right aligned causal mask with seqused_k),
 * causal == 0: to all seq_lens[b] positions.  Keys past the block table's
 * capacity (max_blocks * block_size) are not read.
 *
 * q: total_q x num_q_heads x head_dim (16-byte aligned rows), out likewise
 * (8-byte aligned rows); head_dim 128; num_q_heads / num_kv_heads <= 16;
 * 1..16 centroids per codebook; rot_block 2 or 4.  Other arguments as for
 * rq_int8_prefill.  Every launch size depends only on num_seqs, max_q_len and
 * num_kv_heads, so the call can be captured in a HIP graph.
 */
int rq_paged_attention(const void *q, int32_t dtype, int64_t total_q, int32_t num_q_heads,
                       int64_t q_stride_tok, int64_t q_stride_head,
                       const int32_t *cu_seqlens_q, int64_t num_seqs, int64_t max_q_len, int32_t causal,
                       const uint8_t *kv_cache, int64_t num_blocks, int32_t block_size,
                       int64_t stride_block, int64_t stride_token,
                       int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                       const int32_t *block_table, int64_t max_blocks, int64_t bt_stride_seq,
                       const int32_t *seq_lens,
                       const float *k_centroids, int32_t n_k_centroids,
                       const float *v_centroids, int32_t n_v_centroids,
                       const float *rotation, int32_t rot_block, float sm_scale,
                       void *out, int64_t out_stride_tok, int64_t out_stride_head,
                       void *stream);

/*
 * The non-fused path of rq_paged_attention, same arithmetic, in two launches for
 * long queries: a pack kernel decodes every 64-key tile of every (sequence, kv
 * head) once into a tile image in the workspace (K and V in the q dtype, the
 * values rq_decompress writes; V scaled exactly into fp16 by a power of two),
 * and the attention kernel streams the images (Q K^T on the q dtype's MFMA,
 * exact products and fp32 sums).  rq_paged_attention decodes each tile in
 * every query block's workgroup instead, which suits single-token queries.
 *
 * Replaces the same reference code as rq_paged_attention
 *   src/rotorquant_vllm/vllm/rq_backend.py:937-1036 (non-fused branch).
 * Arguments as for rq_paged_attention, plus max_seq_len (bounds every
 * seq_lens[b]; keys past it are not read) and a workspace of
 * rq_paged_prefill_workspace_bytes() bytes, 16-byte aligned, no initialisation
 * needed.  Centroid counts 1..16.
 */
int rq_paged_prefill(const void *q, int32_t dtype, int64_t total_q, int32_t num_q_heads,
                     int64_t q_stride_tok, int64_t q_stride_head,
                     const int32_t *cu_seqlens_q, int64_t num_seqs, int64_t max_q_len, int32_t causal,
                     const uint8_t *kv_cache, int64_t num_blocks, int32_t block_size,
                     int64_t stride_block, int64_t stride_token,
                     int32_t num_kv_heads, int32_t head_dim, int32_t index_layout,
                     const int32_t *block_table, int64_t max_blocks, int64_t bt_stride_seq,
                     const int32_t *seq_lens, int64_t max_seq_len,
                     const float *k_centroids, int32_t n_k_centroids,
                     const float *v_centroids, int32_t n_v_centroids,
                     const float *rotation, int32_t rot_block, float sm_scale,
                     void *out, int64_t out_stride_tok, int64_t out_stride_head,
                     void *workspace, int64_t workspace_bytes,
                     void *stream);

/* Workspace bytes rq_paged_prefill needs (the same tile images as
 * rq_int8_prefill_workspace_bytes).  No counterpart in the reference, which
 * writes a decompressed copy of every referenced page instead. */
int64_t rq_paged_prefill_workspace_bytes(int64_t num_seqs, int32_t num_kv_heads, int64_t max_seq_len);

#ifdef __cplusplus
}
#endif

#endif /* RQ_ABI_H */
