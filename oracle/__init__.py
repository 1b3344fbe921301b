"""CPU oracle for the speculative-decoding verify path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the ``nanovllm`` package under
``nano-vllm-x_amd/`` or its HIP library) imports this package.  It is used by
``tests/``, ``__graft_entry__.smoke()`` (to check the GPU results) and ``bench.py``'s
``cpu_baseline`` leg (as the timed CPU restatement).

The reference (nano-vllm 0.2.0) has no drafter, tree attention, rejection sampler
or KV compaction.  Each module restates, in numpy float32/int arithmetic, the
reference semantics that do exist and the published algorithm for the rest:

* ``ngram``     -- prompt-lookup drafting with the semantics of transformers'
                   ``PromptLookupCandidateGenerator.get_candidates``
                   (transformers 5.15, generation/candidate_generator.py:1076-1096).
* ``sampler``   -- temperature softmax (reference nanovllm/layers/sampler.py:9-10)
                   and chain/tree rejection sampling (Leviathan et al. 2023 Alg. 1,
                   SpecInfer multi-step residuals) with a fixed fp32 reduction order.
* ``attention`` -- paged attention over the reference KV layout
                   (nanovllm/engine/model_runner.py:115, :151-161, :181) with an
                   ancestor tree mask; the chain tree is the causal bottom-right
                   decode of nanovllm/layers/attention.py:72-74.
* ``kvcache``   -- slot scatter (nanovllm/layers/attention.py:21-30) and accepted
                   path compaction.
* ``draft``     -- the EAGLE draft head's top-k of log_softmax (no reference
                   counterpart; EAGLE-2 tree expansion, arXiv:2406.16858).

How each function is pinned (golden vectors, library cross-checks, closed forms,
brute force) is listed in each module's docstring and exercised in ``tests/``.
"""
