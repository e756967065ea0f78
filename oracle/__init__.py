"""CPU oracle for the paged-KV hot path — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

A restatement of akshajravi/llm-inference-server's algorithms for this path, used
only as the checker: by tests/, by `__graft_entry__.smoke()`, and by bench.py's
`cpu_baseline` leg. Nothing in `llm-inference-server_amd/` imports it, and the HIP
path never routes through it.

Modules (each function cites the reference file:line it restates):

  gather.py  the PyTorch gather attention path, op for op (core/attention.py:92-199),
             and the per-token map (core/attention_triton.py:129-150)
  online.py  the kernel-order online-softmax mirror (core/attention_triton.py:309-384),
             vectorised over heads in numpy float32
  kvops.py   slot arithmetic, KV append, copy-on-write block copy, swap out/in
             (core/block_table.py:137-159, core/paged_executor.py:116-125, 265-270,
             core/kv_pool.py:142-182), in numpy
  greedy.py  greedy sampling over the LM head's logits in the model dtype
             (core/paged_executor.py:194-203), in numpy

How each function is pinned (tests/test_oracle.py): against the reference tests'
closed forms and known answers — the textbook dense causal attention of
tests/test_paged_attention.py:30-37 recomputed in float64, the token-map KAT of
tests/test_paged_attention_triton.py:141-147, the swap round trip of
tests/test_swap.py:35-56, brute-force slot writes, greedy sampling's planted maxima, ties and bf16 rounding
boundaries — and against the committed
golden vectors under tests/golden/. No function here is "parity unpinned".
"""
