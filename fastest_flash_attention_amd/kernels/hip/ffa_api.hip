// C-ABI entry points of libffa.so (declared in include/ffa.h).
//
// Every argument is validated on the host before any HIP call, so malformed calls
// return an error code without touching the device; the kernels themselves then
// only see shapes their grids and bounds checks were written for.

#include <hip/hip_runtime.h>

#include <cmath>

#include "ffa.h"
#include "ffa_common.h"
#include "ffa_internal.h"

namespace {

bool valid_dtype(int32_t dt) { return dt == FFA_DTYPE_BF16 || dt == FFA_DTYPE_FP16; }

// A V narrower than head_dim (taken as zero-padded): the head_dim 192 kernels with
// 128-dim V tiles. FFA_OK, or why the combination is rejected.
int check_v_head_dim(int32_t v_head_dim, int32_t head_dim, int32_t dtype) {
  if (v_head_dim == 0 || v_head_dim == head_dim) return FFA_OK;
  if (!valid_dtype(dtype) || head_dim <= 128 || head_dim > 192 || v_head_dim < 1 || v_head_dim > 128) {
    return FFA_ERR_UNSUPPORTED_HEAD_DIM;
  }
  return v_head_dim % 8 != 0 ? FFA_ERR_MISALIGNED : FFA_OK;
}

// scale: any finite value. softcap: <= 0 (none) or a finite positive cap.
bool valid_scale(float scale, float softcap) {
  return std::isfinite(scale) && !std::isnan(softcap) && !(softcap > 0.0f && std::isinf(softcap));
}

// Every check of a paged decode call except its workspace. *empty: nothing to launch.
int check_decode_args(const ffa_paged_decode_args* a, bool* empty) {
  *empty = false;
  if (a == nullptr) return FFA_ERR_INVALID_ARG;
  if (!valid_dtype(a->dtype)) return FFA_ERR_UNSUPPORTED_DTYPE;
  if (a->head_dim < 1 || a->head_dim > 256) return FFA_ERR_UNSUPPORTED_HEAD_DIM;
  if (a->batch < 0 || a->heads_q < 1 || a->heads_kv < 1 || a->page_size < 1 ||
      a->num_pages < 0 || a->max_context_len < 0 || a->tokens_per_split < 0) {
    return FFA_ERR_INVALID_ARG;
  }
  if (a->heads_q % a->heads_kv != 0) return FFA_ERR_GQA_RATIO;
  if (a->heads_q / a->heads_kv > 64) return FFA_ERR_GQA_RATIO;
  if (a->batch == 0) {
    *empty = true;
    return FFA_OK;
  }
  if (a->q == nullptr || a->o == nullptr || a->k_pages == nullptr || a->v_pages == nullptr ||
      a->block_tables == nullptr || a->context_lens == nullptr) {
    return FFA_ERR_INVALID_ARG;
  }
  const int64_t max_blocks =
      (static_cast<int64_t>(a->max_context_len) + a->page_size - 1) / a->page_size;
  if (a->block_table_stride < max_blocks) return FFA_ERR_INVALID_ARG;
  for (int i = 0; i < 2; ++i) {
    if (a->q_stride[i] < 0 || a->o_stride[i] < 0 || a->lse_stride[i] < 0) {
      return FFA_ERR_INVALID_ARG;
    }
  }
  if (!valid_scale(a->scale, a->softcap)) return FFA_ERR_INVALID_ARG;
  if (a->max_context_len > 0 && a->num_pages < 1) return FFA_ERR_INVALID_ARG;
  // 16-byte loads of q rows, K rows (to registers) and V rows (to LDS)
  if (a->head_dim % 8 != 0) return FFA_ERR_MISALIGNED;
  const void* ptrs[3] = {a->q, a->k_pages, a->v_pages};
  for (const void* ptr : ptrs) {
    if ((reinterpret_cast<uintptr_t>(ptr) & 15u) != 0) return FFA_ERR_MISALIGNED;
  }
  if (a->q_stride[0] % 8 != 0 || a->q_stride[1] % 8 != 0) return FFA_ERR_MISALIGNED;
  return FFA_OK;
}

}  // namespace

extern "C" {

int ffa_abi_version(void) { return FFA_ABI_VERSION; }

const char* ffa_strerror(int status) {
  switch (status) {
    case FFA_OK:
      return "ok";
    case FFA_ERR_INVALID_ARG:
      return "ffa: invalid argument (null pointer, non-positive size, bad stride or "
             "non-finite scale / softcap)";
    case FFA_ERR_UNSUPPORTED_DTYPE:
      return "ffa: unsupported dtype (bfloat16 and float16; float32 for prefill)";
    case FFA_ERR_UNSUPPORTED_HEAD_DIM:
      return "ffa: unsupported head_dim (1..256 supported)";
    case FFA_ERR_MISALIGNED:
      return "ffa: operands must be 16-byte aligned with head_dim and row/head/batch strides "
             "multiples of 8 elements";
    case FFA_ERR_GQA_RATIO:
      return "ffa: heads_q must be a positive multiple of heads_kv";
    case FFA_ERR_WORKSPACE:
      return "ffa: workspace missing or smaller than the entry point's *_workspace_bytes()";
    case FFA_ERR_LAUNCH:
      return "ffa: kernel launch failed";
    case FFA_ERR_NO_DEVICE:
      return "ffa: no usable HIP device";
    case FFA_ERR_TOO_LARGE:
      return "ffa: problem size exceeds 32-bit grid/index limits";
    case FFA_ERR_SCRATCH_LIMIT:
      return "ffa: the split-K partials of this call exceed the allocation-free entry point's "
             "static scratch (FFA_NOALLOC_SCRATCH_BYTES); use ffa_paged_decode_fwd with a "
             "workspace, or longer splits";
    default:
      return "ffa: unknown error";
  }
}

int ffa_prefill_fwd(const ffa_prefill_args* a, void* stream) {
  if (a == nullptr) return FFA_ERR_INVALID_ARG;
  if (!valid_dtype(a->dtype) && a->dtype != FFA_DTYPE_FP32) return FFA_ERR_UNSUPPORTED_DTYPE;
  if (a->head_dim < 1 || a->head_dim > 256) return FFA_ERR_UNSUPPORTED_HEAD_DIM;
  if (const int rc = check_v_head_dim(a->v_head_dim, a->head_dim, a->dtype); rc != FFA_OK) return rc;
  if (a->batch < 0 || a->heads_q < 1 || a->heads_kv < 1 || a->seqlen_q < 0 || a->seqlen_kv < 0) {
    return FFA_ERR_INVALID_ARG;
  }
  if (a->heads_q % a->heads_kv != 0) return FFA_ERR_GQA_RATIO;
  if (a->batch == 0 || a->seqlen_q == 0) return FFA_OK;
  if (a->q == nullptr || a->o == nullptr) return FFA_ERR_INVALID_ARG;
  if (a->seqlen_kv > 0 && (a->k == nullptr || a->v == nullptr)) return FFA_ERR_INVALID_ARG;
  if (a->q_stride[3] != 1 || a->k_stride[3] != 1 || a->v_stride[3] != 1 || a->o_stride[3] != 1) {
    return FFA_ERR_INVALID_ARG;
  }
  for (int i = 0; i < 3; ++i) {
    if (a->q_stride[i] < 0 || a->k_stride[i] < 0 || a->v_stride[i] < 0 || a->o_stride[i] < 0 ||
        a->lse_stride[i] < 0) {
      return FFA_ERR_INVALID_ARG;
    }
  }
  if (!valid_scale(a->scale, a->softcap)) return FFA_ERR_INVALID_ARG;
  // 16-byte vector / direct-to-LDS loads: aligned bases, head_dim and row strides in
  // whole 16-byte chunks.
  if (a->head_dim % 8 != 0) return FFA_ERR_MISALIGNED;
  const void* ptrs[4] = {a->q, a->k, a->v, a->o};
  for (const void* ptr : ptrs) {
    if ((reinterpret_cast<uintptr_t>(ptr) & 15u) != 0) return FFA_ERR_MISALIGNED;
  }
  const int64_t* strides[4] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride};
  for (const int64_t* st : strides) {
    for (int i = 0; i < 3; ++i) {
      if (st[i] % 8 != 0) return FFA_ERR_MISALIGNED;
    }
  }
  if (a->block_key_mask != nullptr) {
    const int64_t need_words = (static_cast<int64_t>(a->seqlen_kv) + 63) / 64;
    if (a->block_visited == nullptr || a->block_key_mask_words < need_words ||
        a->ref_block_q <= 0 || (reinterpret_cast<uintptr_t>(a->block_key_mask) & 7u) != 0) {
      return FFA_ERR_INVALID_ARG;
    }
  }
  // per-tile byte offsets of K/V rows are 32-bit
  if (a->k_stride[2] >= (int64_t{1} << 24) || a->v_stride[2] >= (int64_t{1} << 24)) {
    return FFA_ERR_TOO_LARGE;
  }
  // Positions are int32 inside the kernel.
  const int64_t max_pos = static_cast<int64_t>(a->q_offset) + a->seqlen_q;
  if (max_pos > ffa::kMaxPos || a->seqlen_kv > ffa::kMaxPos || a->q_offset < -ffa::kMaxPos) {
    return FFA_ERR_TOO_LARGE;
  }
  return ffa::launch_prefill(*a, static_cast<hipStream_t>(stream));
}

int ffa_paged_gather(const ffa_paged_gather_args* a, void* stream) {
  if (a == nullptr) return FFA_ERR_INVALID_ARG;
  if (a->elem_bytes != 2 && a->elem_bytes != 4) return FFA_ERR_UNSUPPORTED_DTYPE;
  if (a->heads_kv < 1 || a->page_size < 1 || a->head_dim < 1 || a->context_len < 0 ||
      a->num_pages < 0) {
    return FFA_ERR_INVALID_ARG;
  }
  if (a->context_len == 0) return FFA_OK;
  if (a->k_pages == nullptr || a->v_pages == nullptr || a->k_out == nullptr ||
      a->v_out == nullptr || a->page_table == nullptr) {
    return FFA_ERR_INVALID_ARG;
  }
  return ffa::launch_paged_gather(*a, static_cast<hipStream_t>(stream));
}

int ffa_paged_append(const ffa_paged_append_args* a, void* stream) {
  if (a == nullptr) return FFA_ERR_INVALID_ARG;
  if (a->elem_bytes != 2 && a->elem_bytes != 4) return FFA_ERR_UNSUPPORTED_DTYPE;
  if (a->heads_kv < 1 || a->page_size < 1 || a->head_dim < 1 || a->n_tokens < 0 ||
      a->start < 0 || a->num_pages < 1) {
    return FFA_ERR_INVALID_ARG;
  }
  if (a->n_tokens == 0) return FFA_OK;
  if (a->k_pages == nullptr || a->k_new == nullptr || a->page_table == nullptr) {
    return FFA_ERR_INVALID_ARG;
  }
  // V is optional (K-only pools), but then entirely
  if ((a->v_pages == nullptr) != (a->v_new == nullptr)) return FFA_ERR_INVALID_ARG;
  for (int i = 0; i < 2; ++i) {
    if (a->k_new_stride[i] < 0 || a->v_new_stride[i] < 0) return FFA_ERR_INVALID_ARG;
  }
  if (static_cast<int64_t>(a->start) + a->n_tokens > 0x7fffffff) return FFA_ERR_TOO_LARGE;
  return ffa::launch_paged_append(*a, static_cast<hipStream_t>(stream));
}

int32_t ffa_paged_decode_num_splits(int32_t max_context_len, int32_t tokens_per_split) {
  if (max_context_len < 0) return 0;
  return ffa::decode_num_splits(max_context_len, tokens_per_split);
}

size_t ffa_paged_decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t head_dim,
                                        int32_t max_context_len, int32_t tokens_per_split) {
  if (batch < 0 || heads_q < 0 || head_dim < 0 || max_context_len < 0) return 0;
  return ffa::decode_workspace_bytes(batch, heads_q, head_dim, max_context_len, tokens_per_split);
}

int ffa_paged_decode_fwd(const ffa_paged_decode_args* a, void* stream) {
  bool empty = false;
  const int rc = check_decode_args(a, &empty);
  if (rc != FFA_OK || empty) return rc;
  const size_t need = ffa::decode_workspace_bytes(a->batch, a->heads_q, a->head_dim,
                                                  a->max_context_len, a->tokens_per_split);
  if (need > 0 && (a->workspace == nullptr || a->workspace_bytes < need)) return FFA_ERR_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(a->workspace) & 15u) != 0) return FFA_ERR_MISALIGNED;
  return ffa::launch_paged_decode(*a, static_cast<hipStream_t>(stream));
}

int ffa_paged_decode_fwd_noalloc(const ffa_paged_decode_args* a, void* stream) {
  bool empty = false;
  const int rc = check_decode_args(a, &empty);
  if (rc != FFA_OK || empty) return rc;
  return ffa::launch_paged_decode_noalloc(*a, static_cast<hipStream_t>(stream));
}

size_t ffa_mla_decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t dim_v,
                                      int32_t max_context_len, int32_t tokens_per_split) {
  if (batch < 0 || heads_q < 0 || dim_v < 0 || max_context_len < 0) return 0;
  return ffa::mla_decode_workspace_bytes(batch, heads_q, dim_v, max_context_len,
                                         tokens_per_split);
}

int ffa_mla_decode_fwd(const ffa_mla_decode_args* a, void* stream) {
  if (a == nullptr) return FFA_ERR_INVALID_ARG;
  if (!valid_dtype(a->dtype)) return FFA_ERR_UNSUPPORTED_DTYPE;
  if ((a->dim_v != 256 && a->dim_v != 512) || a->dim_rope != 64) {
    return FFA_ERR_UNSUPPORTED_HEAD_DIM;
  }
  if (a->batch < 0 || a->heads_q < 1 || a->page_size < 1 || a->num_pages < 0 ||
      a->max_context_len < 0 || a->tokens_per_split < 0) {
    return FFA_ERR_INVALID_ARG;
  }
  if (a->batch == 0) return FFA_OK;
  if (a->q == nullptr || a->o == nullptr || a->kv_pages == nullptr ||
      a->block_tables == nullptr || a->context_lens == nullptr) {
    return FFA_ERR_INVALID_ARG;
  }
  const int64_t max_blocks =
      (static_cast<int64_t>(a->max_context_len) + a->page_size - 1) / a->page_size;
  if (a->block_table_stride < max_blocks) return FFA_ERR_INVALID_ARG;
  for (int i = 0; i < 2; ++i) {
    if (a->q_stride[i] < 0 || a->o_stride[i] < 0 || a->lse_stride[i] < 0) {
      return FFA_ERR_INVALID_ARG;
    }
  }
  if (!valid_scale(a->scale, 0.0f)) return FFA_ERR_INVALID_ARG;
  if (a->max_context_len > 0 && a->num_pages < 1) return FFA_ERR_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(a->q) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(a->kv_pages) & 15u) != 0) {
    return FFA_ERR_MISALIGNED;
  }
  if (a->q_stride[0] % 8 != 0 || a->q_stride[1] % 8 != 0) return FFA_ERR_MISALIGNED;
  const size_t need = ffa::mla_decode_workspace_bytes(a->batch, a->heads_q, a->dim_v,
                                                      a->max_context_len, a->tokens_per_split);
  if (need > 0 && (a->workspace == nullptr || a->workspace_bytes < need)) return FFA_ERR_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(a->workspace) & 15u) != 0) return FFA_ERR_MISALIGNED;
  return ffa::launch_mla_decode(*a, static_cast<hipStream_t>(stream));
}

size_t ffa_attn_bwd_workspace_bytes(int32_t batch, int32_t heads_q, int32_t seqlen_q) {
  if (batch < 0 || heads_q < 0 || seqlen_q < 0) return 0;
  return ffa::attn_bwd_workspace_bytes(batch, heads_q, seqlen_q);
}

int ffa_attn_bwd(const ffa_attn_bwd_args* a, void* stream) {
  if (a == nullptr) return FFA_ERR_INVALID_ARG;
  if (!valid_dtype(a->dtype) && a->dtype != FFA_DTYPE_FP32) return FFA_ERR_UNSUPPORTED_DTYPE;
  if (a->head_dim < 1 || a->head_dim > 256) return FFA_ERR_UNSUPPORTED_HEAD_DIM;
  if (const int rc = check_v_head_dim(a->v_head_dim, a->head_dim, a->dtype); rc != FFA_OK) return rc;
  if (a->batch < 0 || a->heads_q < 1 || a->heads_kv < 1 || a->seqlen_q < 0 || a->seqlen_kv < 0) {
    return FFA_ERR_INVALID_ARG;
  }
  if (a->heads_q % a->heads_kv != 0) return FFA_ERR_GQA_RATIO;
  if (a->batch == 0 || a->seqlen_q == 0) return FFA_OK;
  if (a->dout == nullptr || a->q == nullptr || a->o == nullptr || a->lse == nullptr ||
      a->dq == nullptr) {
    return FFA_ERR_INVALID_ARG;
  }
  if (a->seqlen_kv > 0 && (a->k == nullptr || a->v == nullptr || a->dk == nullptr ||
                           a->dv == nullptr)) {
    return FFA_ERR_INVALID_ARG;
  }
  const int64_t* strides[8] = {a->do_stride, a->q_stride,  a->k_stride,  a->v_stride,
                               a->o_stride,  a->dq_stride, a->dk_stride, a->dv_stride};
  for (const int64_t* st : strides) {
    if (st[3] != 1) return FFA_ERR_INVALID_ARG;
    for (int i = 0; i < 3; ++i) {
      if (st[i] < 0) return FFA_ERR_INVALID_ARG;
    }
  }
  for (int i = 0; i < 3; ++i) {
    if (a->lse_stride[i] < 0) return FFA_ERR_INVALID_ARG;
  }
  if (!valid_scale(a->scale, a->softcap)) return FFA_ERR_INVALID_ARG;
  if (a->head_dim % 8 != 0) return FFA_ERR_MISALIGNED;
  const void* ptrs[8] = {a->dout, a->q, a->k, a->v, a->o, a->dq, a->dk, a->dv};
  for (const void* ptr : ptrs) {
    if ((reinterpret_cast<uintptr_t>(ptr) & 15u) != 0) return FFA_ERR_MISALIGNED;
  }
  for (const int64_t* st : strides) {
    for (int i = 0; i < 3; ++i) {
      if (st[i] % 8 != 0) return FFA_ERR_MISALIGNED;
    }
  }
  // 32-bit byte offsets of rows inside a tile
  if (a->q_stride[2] >= (int64_t{1} << 24) || a->do_stride[2] >= (int64_t{1} << 24) ||
      a->k_stride[2] >= (int64_t{1} << 24) || a->v_stride[2] >= (int64_t{1} << 24)) {
    return FFA_ERR_TOO_LARGE;
  }
  const int64_t max_pos = static_cast<int64_t>(a->q_offset) + a->seqlen_q;
  if (max_pos > ffa::kMaxPos || a->seqlen_kv > ffa::kMaxPos || a->q_offset < -ffa::kMaxPos) {
    return FFA_ERR_TOO_LARGE;
  }
  const size_t need = ffa::attn_bwd_workspace_bytes(a->batch, a->heads_q, a->seqlen_q);
  if (a->workspace == nullptr || a->workspace_bytes < need) return FFA_ERR_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(a->workspace) & 15u) != 0) return FFA_ERR_MISALIGNED;
  return ffa::launch_attn_bwd(*a, static_cast<hipStream_t>(stream));
}

}  // extern "C"
