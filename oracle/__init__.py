"""CPU oracle of the forward attention hot path — TEST INFRASTRUCTURE ONLY.

The checker against which the HIP kernels are judged. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it;
``fastest_flash_attention_amd`` never does and has no CPU path.

Modules (each cites the reference file:line it restates):
  reference_forward  flash_attn_cpu_forward + dispatcher CPU branch (numpy fp32)
  naive              fp64 brute-force masked SDPA (pins reference_forward)
  paged              PagedKVCache index law, get_kv gather, decode oracle
  block_masks        block-sparse mask generators, tiles visited per query tile
  caches             ContinuousKVCache

Parity pinning status (tests/test_oracle.py): every function above is pinned; see
the module docstrings for what pins each.
"""
