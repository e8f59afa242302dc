"""CPU oracle of the packed attention forward. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg import this package, and only as
the checker (or the timed CPU baseline); the product (``karpo_decision_amd``) never imports, calls or falls back to it.

Modules:
  attention  the reference's torch attention path restated: per-sequence SDPA with the varlen mask contract
  brute      float64 loops over (query, head, key) for tiny cases, stated rule by rule
  schedule   brute-force enumeration of allowed pairs and of each query tile's key-step envelope

Pinning (which checks fix each function; tests/test_oracle.py and tests/test_plan.py):
  attention.visible        the reference's mask formulas as literal known-answer sets (window edges, alignment, spans),
                           and brute.visible on random layouts
  attention.packed_attention  brute.attention (float64) on random packs; closed forms: q = 0 gives the mean of the
                           visible values; one-hot values reveal the mask; two keys give a logistic weight; GQA head
                           mapping by constant per-head values; golden fixtures in tests/golden
  brute.attention          the same closed forms and the golden fixtures
  schedule.*               pair counts in closed form (L(L+1)/2, window and span formulas) and the tiny workload's
                           184,925 pairs
"""
