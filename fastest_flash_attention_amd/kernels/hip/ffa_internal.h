// Internal launch interface between the C-ABI layer (ffa_api.hip) and the kernel
// translation units. Arguments arrive here already validated.
#pragma once

#include <hip/hip_runtime.h>

#include "ffa.h"

namespace ffa {

// Prefill: one launch of the fused forward kernel.
int launch_prefill(const ffa_prefill_args& a, hipStream_t stream);

// Paged decode: split kernel + logsumexp combine kernel.
int32_t decode_num_splits(int32_t max_context_len, int32_t tokens_per_split);
int32_t decode_tokens_per_split(int32_t tokens_per_split);
size_t decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t head_dim,
                              int32_t max_context_len, int32_t tokens_per_split);
int launch_paged_decode(const ffa_paged_decode_args& a, hipStream_t stream);
// The same launch with the split-K partials in the library's static scratch array.
int launch_paged_decode_noalloc(const ffa_paged_decode_args& a, hipStream_t stream);

// MLA decode over the compressed latent cache: split kernel + the decode combine kernel.
int32_t mla_decode_tokens_per_split(int32_t tokens_per_split);
int32_t mla_decode_num_splits(int32_t max_context_len, int32_t tokens_per_split);
size_t mla_decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t dim_v,
                                  int32_t max_context_len, int32_t tokens_per_split);
int launch_mla_decode(const ffa_mla_decode_args& a, hipStream_t stream);

// Attention backward: preprocess, dK/dV and dQ kernels.
size_t attn_bwd_workspace_bytes(int32_t batch, int32_t heads_q, int32_t seqlen_q);
int launch_attn_bwd(const ffa_attn_bwd_args& a, hipStream_t stream);

// get_kv gather.
int launch_paged_gather(const ffa_paged_gather_args& a, hipStream_t stream);
int launch_paged_append(const ffa_paged_append_args& a, hipStream_t stream);

}  // namespace ffa
