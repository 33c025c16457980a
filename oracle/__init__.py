"""CPU oracle of the paged-attention path — TEST INFRASTRUCTURE ONLY.

Restates the reference's algorithm (nvivek17/NitroRAG src/model_q8.cpp
attention loops, src/pagedMemory.hpp page bookkeeping) so the HIP path can be
checked against it.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this package, and only to check results against
or as the timed CPU baseline; the shipped library (nitrorag_amd) never does.

Modules:
  attn          ctypes wrappers over the C restatement (attn_oracle.c)
  paged_memory  pure-Python restatement of KVBlock_Manager / PrefixCacheManager / Sequence
  closed_form   fp64 softmax(qK^T/sqrt(hd))V over block-table-resolved rows
  ref           driver of the reference's own compiled code (this container only)
"""
