"""CPU oracle for the GQA decode-attention hot path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as the
checker (or, for cpu_baseline, as the timed CPU restatement of the reference's PyTorch path). The product path
(the breeze-tts-2-flash_amd package and libbz_gqa_decode.so) never calls it and has no CPU fallback.

Modules:
  bf16       bf16 <-> fp32 bit conversions (round to nearest even), numpy uint16 storage
  attention  the attention restatements:
               decode_attention      parity oracle: exact softmax attention, float64, KV heads expanded, sliced to
                                     [start, end) per row (north star: fp32 SDPA with expanded KV heads)
               sdpa_fp32             the same through torch's scaled_dot_product_attention in fp32 (CPU)
               eager_bf16            the reference's eager rounding chain (models/breeze.py:259-286) in torch on the
                                     CPU: the CPU baseline's code under test
               mask_interval / interval_mask   the reference's interval mask (backbone_graph.py:239-252)

Pins (tests/test_oracle.py): bf16 conversion against torch's bf16 cast; decode_attention against torch SDPA, a
pure-Python float64 brute force on tiny shapes, closed forms (one position -> v[start]; q = 0 or scale = 0 -> mean
of V over the range; one dominant key -> its V row), invariants (GQA == MHA on expanded K/V, NaN outside the range
never reaches the output, row independence), and planted mistakes (wrong head map, off-by-one range, missing scale)
that those checks must reject. The reference has no golden vectors of its own for this path.
"""
