"""CPU oracle of sglang-neuron's paged decode-attention path. TEST INFRASTRUCTURE ONLY.

This package restates the reference's PyTorch path in plain torch (CPU) and numpy, function by function, each citing
the reference file:line it follows. It is the checker that the HIP path is compared with.

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of bench.py may import it. It is never the
thing measured or shipped: the product path (sglang_neuron_amd) does not import it and has no CPU fallback.

How each function is pinned (tests/test_oracle_*.py):
  fp8      torch's float -> float8_e4m3fn cast, which the store restatement uses, is checked against a
           nearest-value search over the 255 finite e4m3fn values built from the OCP definition. The check covers
           all 65,536 bf16 patterns at several scales, plus the reference's own known answer
           quantize_fp8_e4m3fn([1.1, 500.0]) -> [1.125, 448.0] (models/kimi_k3/kernels/decode/mla_decode_torch.py:
           89-96).
  store    slot arithmetic (page, head, offset), out-of-pool redirection to slot 0, bytes untouched outside the
           written slots; the DSA byte map against the reference docstring's bijection (kv_row_layout.py:62-84).
  attention float64 brute force with explicit loops on tiny inputs; closed forms (one key -> its value, equal keys
           -> the mean of the values, a -inf sink -> no sink, a window >= L -> full attention, an index list of
           every prior position -> dense MLA, FP8 with scale 1 on representable values -> the bf16 result); page
           permutation invariance; split + LSE merge == unsplit.
  metadata brute-force construction of the block table from req_to_token.
  indexer  the key cast against the e4m3fn definition and a known answer; the score by explicit float64 loops;
           the top-k against a full sort.
  page_items the item address against the pools' tensor indexing; pack by byte loops; unpack(pack) and
           copy == unpack(pack) invariants.
  qkv      RoPE at angle 0 is the identity and at a quarter turn the exact rotate-half; RoPE against complex
           multiplication in float64 within its three bf16 roundings; RMSNorm of a constant-magnitude head against
           its closed form; the writes against the pinned MHA store.
Nothing here is "parity unpinned"; see the tests for the pin of each function.
"""
