/*
 * ffa.h — C ABI of the MI355X (gfx950) forward-attention library `libffa.so`.
 *
 * Plain C: pointers, sizes and one POD argument struct per entry point. No torch
 * or HIP types cross this boundary (the stream is passed as `void*` holding a
 * `hipStream_t`). The caller owns every buffer, including the split-K workspace
 * of paged decode; the library allocates nothing on these paths and launches
 * asynchronously on the given stream. Every entry point returns FFA_OK (0) or a
 * negative ffa_status; exceptions never cross the ABI. Entry points are stateless
 * and reentrant.
 *
 * Reference interfaces replaced (paths relative to MindIntels/fastest_flash_attention):
 *   ffa_prefill_fwd        <- ffpa_attn_triton_forward   kernels/triton_ffpa.py:217-306
 *                             flash_attn_triton_forward  kernels/triton_fwd.py:144-224
 *                             (both reached from the GPU branch of
 *                              ops/attention_forward.py:112-143; the CPU branch
 *                              flash_attn_cpu_forward kernels/cpu_reference.py:132-312
 *                              defines the semantics)
 *   ffa_paged_gather       <- PagedKVCache.get_kv        ops/kv_cache.py:208-232
 *   ffa_paged_decode_fwd   <- PagedKVCache.get_kv + fastest_flash_attn_forward(S_q=1)
 *                             ops/kv_cache.py:208-232, ops/attention_forward.py:23-167
 *   ffa_paged_decode_workspace_bytes, ffa_paged_decode_num_splits: sizing helpers of
 *                             the decode entry point (no reference counterpart; the
 *                             reference has no fused decode).
 *   ffa_mla_decode_fwd     <- FastestFlashMLA attention for one new token
 *                             (modules/flash_mla.py:116-172, reached with the up-projected
 *                              K/V of all previous tokens as kv_cache): the reference has
 *                              no MLA decode path; this one reads the compressed latent
 *                              cache instead of up-projected K/V.
 *   ffa_mla_decode_workspace_bytes: sizing helper of the MLA decode entry point.
 *   ffa_attn_bwd           <- fastest_flash_attn_backward   ops/attention_backward.py:19-76
 *                             (its GPU branch flash_attn_triton_backward
 *                              kernels/triton_bwd.py:122-190; the CPU branch
 *                              flash_attn_cpu_backward kernels/cpu_reference.py:319-427
 *                              defines the semantics), reached from
 *                             FastestFlashAttnFunc.backward ops/attention_func.py:61-90.
 *   ffa_attn_bwd_workspace_bytes: sizing helper of the backward entry point.
 *   ffa_strerror, ffa_abi_version: error text / version probe, replacing the
 *                             availability probe check_triton_available utils.py:20-29.
 */
#ifndef FFA_H_
#define FFA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FFA_ABI_VERSION 7

typedef enum ffa_status {
  FFA_OK = 0,
  FFA_ERR_INVALID_ARG = -1,      /* null pointer, non-positive size, bad stride,
                                    non-finite scale or softcap, ... */
  FFA_ERR_UNSUPPORTED_DTYPE = -2,
  FFA_ERR_UNSUPPORTED_HEAD_DIM = -3,
  FFA_ERR_MISALIGNED = -4,       /* base not 16-byte aligned, or head_dim / a stride not a
                                    multiple of 8 elements (prefill) */
  FFA_ERR_GQA_RATIO = -5,        /* heads_q not a multiple of heads_kv */
  FFA_ERR_WORKSPACE = -6,        /* workspace missing or too small */
  FFA_ERR_LAUNCH = -7,           /* hipGetLastError() reported a launch failure */
  FFA_ERR_NO_DEVICE = -8,        /* no usable HIP device / device query failed */
  FFA_ERR_TOO_LARGE = -9,        /* a size exceeds what the kernels index with 32 bits */
  FFA_ERR_SCRATCH_LIMIT = -10    /* ffa_paged_decode_fwd_noalloc: the call's split-K
                                    partials exceed FFA_NOALLOC_SCRATCH_BYTES */
} ffa_status;

typedef enum ffa_dtype {
  FFA_DTYPE_BF16 = 0,
  FFA_DTYPE_FP16 = 1,
  FFA_DTYPE_FP32 = 2   /* ffa_prefill_fwd (fp32 MFMA) and ffa_attn_bwd (fp32 FMA) only */
} ffa_dtype;

/*
 * Prefill / general forward attention.
 *
 * Semantics (kernels/cpu_reference.py:132-312, ops/attention_forward.py:23-167):
 *   S      = (q . k^T) * scale                       fp32 accumulation; scale is any
 *            finite value, as the replaced launchers accept (a negative scale gives
 *            the softmax of the negated scores, zero the uniform softmax over the
 *            visible keys with lse = log(n)); a non-finite scale is FFA_ERR_INVALID_ARG
 *   S      = softcap * tanh(S / softcap)              if softcap > 0, before masking
 *   masked : key >= seqlen_kv,
 *            causal && key > q_offset + row,          (top-left aligned when q_offset=0)
 *            window > 0 && key < q_offset + row - window + 1   (one-sided if !causal)
 *   O      = softmax(S) . v   (rows with no visible key: O = 0)
 *   lse    = natural-log logsumexp of the visible S of the row, fp32.
 *            A row with no visible key gets the reference's sentinel
 *            log(n * 1e-30), n = number of (ref_block_q x ref_block_kv) tiles the
 *            reference loop visits for that row (-inf when n == 0, and always -inf
 *            with masked_lse_mode = 1).
 * Block sparsity (the reference's block_mask, cpu_reference.py:220-222): when
 * block_key_mask is not NULL, key k is also masked for row r unless bit (k % 64) of
 * block_key_mask[(r / ref_block_q) * block_key_mask_words + k / 64] is set (the
 * [n_br, n_bc] tile mask expanded to keys: bit k of row-block i = block_mask[i][k /
 * ref_block_kv]); block_visited[r / ref_block_q] then gives the sentinel's n.
 * GQA: q head h reads kv head h / (heads_q / heads_kv)  (utils.py:111-130).
 * Layout: element strides per tensor in order [batch, head, seq, dim]; the dim
 * stride must be 1. A batch or head stride may be 0 (broadcast). lse strides are
 * [batch, head, seq]. q/k/v/o share the dtype (bf16 / fp16 on bf16 / fp16 MFMA with
 * fp32 softmax and accumulation; fp32 on fp32 MFMA). q/k/v/o are 16-byte aligned, head_dim
 * and the batch/head/seq strides are multiples of 8 elements (FFA_ERR_MISALIGNED
 * otherwise), and k/v seq strides are below 2^24 elements. Positions are 32-bit in the
 * kernels: |q_offset|, q_offset + seqlen_q and seqlen_kv must not exceed 2^29 - 1
 * (FFA_ERR_TOO_LARGE; the same for ffa_attn_bwd).
 */
typedef struct ffa_prefill_args {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;               /* NULL: do not write LSE */
  int64_t q_stride[4];
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t o_stride[4];
  int64_t lse_stride[3];
  int32_t batch;
  int32_t heads_q;
  int32_t heads_kv;
  int32_t seqlen_q;
  int32_t seqlen_kv;
  int32_t head_dim;         /* 1..256 */
  int32_t q_offset;         /* absolute position of query row 0 */
  int32_t causal;           /* 0 / 1 */
  int32_t window;           /* <= 0: no sliding window */
  float scale;              /* any finite value */
  float softcap;            /* <= 0: no softcap; else finite */
  int32_t ref_block_q;      /* reference tile sizes: only used for the LSE sentinel */
  int32_t ref_block_kv;     /*   of rows with no visible key; <= 0 means 64 */
  int32_t masked_lse_mode;  /* 0: one-pass sentinel log(n*1e-30); 1: -inf (the
                               reference's two_pass LSE, cpu_reference.py:63-125) */
  int32_t dtype;            /* ffa_dtype */
  const uint64_t* block_key_mask;  /* NULL: no block mask; else [n_br][words] bits */
  int32_t block_key_mask_words;    /* words per row block, >= ceil(seqlen_kv / 64) */
  const int32_t* block_visited;    /* [n_br] reference tiles visited per row block
                                      (required with block_key_mask) */
  int32_t v_head_dim;  /* 0 or head_dim: v has head_dim dims. Otherwise v (and its
                          strides) has v_head_dim < head_dim dims and is taken as
                          zero-padded to head_dim: O dims >= v_head_dim are written 0,
                          the result the reference gives for the zero-padded V that the
                          MLA module builds (modules/flash_mla.py:151-152). Supported for
                          bf16 / fp16 at head_dim 129..192 with v_head_dim <= 128, a
                          multiple of 8 (FFA_ERR_UNSUPPORTED_HEAD_DIM otherwise). */
} ffa_prefill_args;

int ffa_prefill_fwd(const ffa_prefill_args* args, void* stream);

/*
 * Paged KV pool, layout of PagedKVCache (ops/kv_cache.py:142-149):
 *   k_pages, v_pages : [num_pages, heads_kv, page_size, head_dim], contiguous.
 * Index law (ops/kv_cache.py:194-203): token t of sequence b lives in physical
 * page block_tables[b * block_table_stride + t / page_size], slot t % page_size.
 * Page ids outside [0, num_pages) never address memory. The reference raises
 * IndexError for them (ops/kv_cache.py:226-227); here, in the decode entry points,
 * the tokens such an id would hold are excluded from the attention, exactly like
 * tokens past context_len (a sequence left with no token gets O = 0, lse = -inf);
 * ffa_paged_gather writes zeros for them and ffa_paged_append skips them. Callers
 * that want the reference's error check the ids first (the Python layer offers
 * that check as an option).
 */

/* Gather sequence pages into contiguous [heads_kv, context_len, head_dim] (get_kv). */
typedef struct ffa_paged_gather_args {
  const void* k_pages;
  const void* v_pages;
  void* k_out;              /* [heads_kv, context_len, head_dim] contiguous */
  void* v_out;
  const int32_t* page_table;/* device, >= ceil(context_len / page_size) entries */
  int32_t num_pages;        /* pool size, for bounds of page ids */
  int32_t heads_kv;
  int32_t page_size;
  int32_t head_dim;
  int32_t context_len;
  int32_t elem_bytes;       /* 2 or 4 */
} ffa_paged_gather_args;

int ffa_paged_gather(const ffa_paged_gather_args* args, void* stream);

/*
 * Append n_tokens new tokens to one sequence (PagedKVCache.append_tokens,
 * ops/kv_cache.py:170-206): token t of the new block is token start + t of the
 * sequence and goes to page page_table[(start + t) / page_size], slot
 * (start + t) % page_size, for every KV head. The caller has allocated the pages
 * (page_table holds >= ceil((start + n_tokens) / page_size) valid ids, each in
 * [0, num_pages); FFA_ERR_INVALID_ARG is not detected on the device for bad ids,
 * which are skipped). k_new / v_new are [heads_kv, n_tokens, head_dim] with element
 * strides new_stride[head, token] (dim stride 1) and the pool's dtype. v_pages and v_new
 * may both be NULL: a K-only append (the MLA latent pool, one row per token).
 */
typedef struct ffa_paged_append_args {
  void* k_pages;
  void* v_pages;
  const void* k_new;
  const void* v_new;
  const int32_t* page_table;  /* device, the sequence's page table */
  int64_t k_new_stride[2];
  int64_t v_new_stride[2];
  int32_t num_pages;
  int32_t heads_kv;
  int32_t page_size;
  int32_t head_dim;
  int32_t start;              /* tokens already stored for the sequence */
  int32_t n_tokens;
  int32_t elem_bytes;         /* 2 or 4 */
} ffa_paged_append_args;

int ffa_paged_append(const ffa_paged_append_args* args, void* stream);

/*
 * Batched paged decode: one query token per sequence, attending to the first
 * context_lens[b] tokens of sequence b. The query sits at absolute position
 * context_lens[b]-1, i.e. the reference call
 *   fastest_flash_attn_forward(q[b:b+1,:,None], K, V, num_kv_heads=Hkv,
 *                              kv_cache=(K[:, :, :L-1], V[:, :, :L-1]) ...)
 * with K, V = get_kv(seq b): every cached key is visible, a sliding window keeps
 * keys >= L - window, softcap as in prefill.
 *   q   : [batch, heads_q, head_dim] (strides q_stride[b, h], dim stride 1)
 *   o   : [batch, heads_q, head_dim] (strides o_stride[b, h])
 *   lse : [batch, heads_q] fp32 (strides lse_stride[b, h]) or NULL
 * context_lens[b] == 0 gives O = 0 and lse = -inf. head_dim % 8 == 0; q, the pools and
 * the workspace are 16-byte aligned and q's strides are multiples of 8
 * (FFA_ERR_MISALIGNED). tokens_per_split is rounded up to a multiple of 16 and clamped
 * to [32, 2048]; ceil(max_context_len / tokens_per_split) must not exceed 65535
 * (FFA_ERR_TOO_LARGE).
 * Split-K: each sequence is cut into chunks of tokens_per_split tokens processed
 * by independent workgroups; partials (O, lse) go to the caller's workspace and
 * are merged by logsumexp weights.
 */
typedef struct ffa_paged_decode_args {
  const void* q;
  const void* k_pages;
  const void* v_pages;
  void* o;
  float* lse;
  const int32_t* block_tables;   /* [batch, block_table_stride] int32 */
  const int32_t* context_lens;   /* [batch] int32 */
  void* workspace;
  size_t workspace_bytes;
  int64_t q_stride[2];
  int64_t o_stride[2];
  int64_t lse_stride[2];
  int32_t block_table_stride;
  int32_t batch;
  int32_t heads_q;
  int32_t heads_kv;
  int32_t head_dim;              /* 1..256 */
  int32_t page_size;
  int32_t num_pages;
  int32_t max_context_len;       /* upper bound of context_lens (sizes the grid) */
  int32_t tokens_per_split;      /* 0: library default */
  int32_t window;                /* <= 0: none */
  float scale;                   /* any finite value */
  float softcap;                 /* <= 0: none; else finite */
  int32_t dtype;                 /* FFA_DTYPE_BF16 or FFA_DTYPE_FP16 */
} ffa_paged_decode_args;

/* Split count per sequence the decode entry point uses for these sizes. */
int32_t ffa_paged_decode_num_splits(int32_t max_context_len, int32_t tokens_per_split);
/* Workspace bytes needed by ffa_paged_decode_fwd for these sizes. */
size_t ffa_paged_decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t head_dim,
                                        int32_t max_context_len, int32_t tokens_per_split);
int ffa_paged_decode_fwd(const ffa_paged_decode_args* args, void* stream);

/*
 * Allocation-free paged decode. It has no counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments, semantics, kernels
 * and results as ffa_paged_decode_fwd, except that args->workspace and
 * args->workspace_bytes are ignored: the split-K partials go to a library-owned
 * device array of FFA_NOALLOC_SCRATCH_BYTES, one per GPU the library runs on, held
 * until the process ends. A call whose ffa_paged_decode_workspace_bytes() exceeds it
 * returns FFA_ERR_SCRATCH_LIMIT (fewer, longer splits need less). No memory is
 * allocated or freed. Every call on one GPU shares that GPU's array and leaves its
 * partials there: calls that overlap on one GPU (other streams, other threads) race,
 * so the caller serialises them. Nothing in the array has to start at zero (each
 * call writes every partial it reads). The first call on a device looks up the
 * array's address on that device once (hipGetSymbolAddress): make that first call
 * eagerly, outside HIP graph capture; later calls may be captured and replayed.
 * The array is a standing cost: loading libffa.so reserves its 64 MiB on every GPU
 * where the code object is loaded, whether or not this entry point is ever called.
 */
#define FFA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int ffa_paged_decode_fwd_noalloc(const ffa_paged_decode_args* args, void* stream);

/*
 * MLA decode over the compressed latent cache (no counterpart in the reference, which
 * up-projects K/V per head; see FastestFlashMLA, modules/flash_mla.py:116-172). Every
 * query head attends over one shared row per token,
 *   kv_pages : [num_pages, page_size, dim_v + dim_rope], contiguous: the latent c_t
 *              (dim_v) followed by the rotated k_rope r_t (dim_rope),
 * with the absorbed query q_h = [W_uk_h^T q_nope_h, q_rope_h] and V = the first dim_v
 * dims of the row. Scores are scale * q_h . row_t over the first context_lens[b] tokens
 * (page index law as for the paged pools); the output is the latent-space
 * O_lat_h = sum_t p_t c_t, which the caller up-projects with W_uv_h.
 *   q   : [batch, heads_q, dim_v + dim_rope] (strides q_stride[b, h], dim stride 1)
 *   o   : [batch, heads_q, dim_v] (strides o_stride[b, h])
 *   lse : [batch, heads_q] fp32 (strides lse_stride[b, h]) or NULL
 * dim_v is 256 or 512 and dim_rope is 64 (FFA_ERR_UNSUPPORTED_HEAD_DIM). q and
 * kv_pages are 16-byte aligned, q's strides multiples of 8 (FFA_ERR_MISALIGNED).
 * tokens_per_split (0: library default 512) is rounded up to a multiple of 32 and
 * capped at 1024, and ceil(max_context_len / tokens_per_split) must not exceed 65535
 * (FFA_ERR_TOO_LARGE); split-K partials go to the workspace: normalised O partials in
 * the input's 16-bit type (a convex combination of latent rows is representable there)
 * and one fp32 lse per (sequence, head, split), merged as in ffa_paged_decode_fwd.
 */
typedef struct ffa_mla_decode_args {
  const void* q;
  const void* kv_pages;
  void* o;
  float* lse;
  const int32_t* block_tables;   /* [batch, block_table_stride] int32 */
  const int32_t* context_lens;   /* [batch] int32 */
  void* workspace;
  size_t workspace_bytes;
  int64_t q_stride[2];
  int64_t o_stride[2];
  int64_t lse_stride[2];
  int32_t block_table_stride;
  int32_t batch;
  int32_t heads_q;
  int32_t dim_v;                 /* 256 or 512 */
  int32_t dim_rope;              /* 64 */
  int32_t page_size;
  int32_t num_pages;
  int32_t max_context_len;
  int32_t tokens_per_split;      /* 0: library default */
  float scale;                   /* any finite value */
  int32_t dtype;                 /* FFA_DTYPE_BF16 or FFA_DTYPE_FP16 */
} ffa_mla_decode_args;

size_t ffa_mla_decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t dim_v,
                                      int32_t max_context_len, int32_t tokens_per_split);
int ffa_mla_decode_fwd(const ffa_mla_decode_args* args, void* stream);

/*
 * Attention backward (recompute): gradients of the prefill forward above for one
 * upstream gradient dO, from q, k, v, the forward's O and its natural-log LSE.
 * Semantics (kernels/cpu_reference.py:319-427):
 *   P   = exp(S - lse)  with S, the masks and softcap as in ffa_prefill_fwd
 *         (a row with lse = -inf has P = 0)
 *   D_i = sum_d dO[i, d] * O[i, d]                    fp32
 *   dV  = P^T dO
 *   dS  = P * (dO V^T - D_i), times 1 - tanh^2(q.k * scale / softcap) with softcap
 *   dQ  = scale * dS K,   dK = scale * dS^T Q
 * GQA: dK / dV of kv head j sum over the q heads j * ratio .. (j + 1) * ratio - 1.
 * Layout: element strides [batch, head, seq, dim] (dim stride 1; dq/dk/dv written in
 * place, no broadcast strides on them); lse strides [batch, head, seq]. All of dout,
 * q, k, v, o, dq, dk, dv share the dtype: bf16 / fp16 (MFMA with fp32 accumulation, P
 * and dS rounded to the dtype for the matrix products) or fp32 (fp32 FMAs throughout,
 * as the reference computes fp32 inputs). head_dim is 1..256 and a multiple of
 * 8; every tensor is 16-byte aligned with batch/head/seq strides multiples of 8
 * elements (FFA_ERR_MISALIGNED) and seq strides below 2^24 elements. The workspace
 * (16-byte aligned, ffa_attn_bwd_workspace_bytes()) holds per-row statistics; the
 * call overwrites all of it. Three kernels, no atomics: results do not depend on
 * scheduling.
 */
typedef struct ffa_attn_bwd_args {
  const void* dout;
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const float* lse;
  void* dq;
  void* dk;
  void* dv;
  void* workspace;
  size_t workspace_bytes;
  int64_t do_stride[4];
  int64_t q_stride[4];
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t o_stride[4];
  int64_t dq_stride[4];
  int64_t dk_stride[4];
  int64_t dv_stride[4];
  int64_t lse_stride[3];
  int32_t batch;
  int32_t heads_q;
  int32_t heads_kv;
  int32_t seqlen_q;
  int32_t seqlen_kv;
  int32_t head_dim;         /* 1..256 */
  int32_t q_offset;
  int32_t causal;
  int32_t window;           /* <= 0: no sliding window */
  float scale;              /* any finite value */
  float softcap;            /* <= 0: no softcap; else finite */
  int32_t dtype;            /* ffa_dtype */
  int32_t v_head_dim;       /* 0 or head_dim: v and dv have head_dim dims. Otherwise v
                               and dv have v_head_dim < head_dim dims, v taken as
                               zero-padded to head_dim as in ffa_prefill_fwd (dout and o
                               keep head_dim dims); the same support rule. */
} ffa_attn_bwd_args;

size_t ffa_attn_bwd_workspace_bytes(int32_t batch, int32_t heads_q, int32_t seqlen_q);
int ffa_attn_bwd(const ffa_attn_bwd_args* args, void* stream);

const char* ffa_strerror(int status);
int ffa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FFA_H_ */
