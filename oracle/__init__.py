"""Oracle for the nano-inference attention path - TEST INFRASTRUCTURE ONLY.

This package checks the HIP path; it is never the thing measured or shipped.  Only the
tests, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import it.  The product path (``nano_inference_amd``) never imports it and
fails loudly when its HIP library is missing.

Modules
  reference_attention  op-for-op PyTorch-CPU restatement of the reference's
                       attention (src/nano_inference/layers/attention.py:12-50,
                       :267-332; layers/vision.py:190-208).  Also the timed CPU
                       baseline.
  textbook             independent float64 numpy attention (softmax(qK^T s)V per
                       row with an explicit visible-key bound) plus a pure-Python
                       brute force for tiny inputs; the numeric oracle of the
                       GPU parity tests.
  metadata             restatement of the context builder's slot mapping, block
                       tables, context lengths and mask
                       (src/nano_inference/engine/context_builder.py:83-193).
  vision_windows       restatement of the ViT window permutation and cu_seqlens
                       (src/nano_inference/layers/vision.py:365-412, :443-453).
  qk_rope              op-for-op restatement of QK-RMSNorm and RoPE / mRoPE
                       (layers/norm.py:35-47, layers/rotary.py:8-33, :105-130,
                       :184-210), the steps in front of the KV write.

Pinning (what checks each function; see tests/test_oracle_*.py)
  reference_attention.sdpa          torch.nn.functional.scaled_dot_product_attention
                                    (library), textbook, brute force; causality
                                    invariant of tests/unit/test_attention.py:16-33.
  reference_attention.kv_write_loop closed-form destination index; KAT slots of
                                    tests/unit/test_context_builder.py:48-58, :87.
  reference_attention.paged_*       textbook on gathered keys; block-table permutation
                                    invariance; GQA == MHA with repeated KV; garbage
                                    past the context has no effect; closed forms
                                    (L=1 -> v0, equal keys -> mean V, constant V).
  textbook.*                        brute force on tiny inputs; closed forms; a planted
                                    mistake (wrong GQA map, dropped scale) must fail.
  metadata.*                        KATs of tests/unit/test_context_builder.py.
  qk_rope.*                         KATs and properties of tests/unit/test_norm.py,
                                    test_rotary.py, test_mrope.py; closed-form rotation
                                    of unit vectors; relative-position invariance in
                                    float64; planted mistakes (sign, pairing, section)
                                    must fail.
  vision_windows.*                  135 windows / 7528 tokens / <=64 tokens per window
                                    for the 4-image grid; brute-force window enumeration.
"""
