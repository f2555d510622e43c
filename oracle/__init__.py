"""CPU oracle for the k8v4 quantized paged-KV attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package may import this
package; only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` use it, and only as the reference results a kernel is
compared with or as the timed CPU baseline.

It restates, independently of the product code, the reference's rules:

* ``quant``     -- K int8 / V affine int4 quantization in float64
                   (k8v4_v030/oracle.py:18-77);
* ``scalar``    -- a pure-Python scalar restatement of the same rules and of
                   ``causal_gqa`` for tiny cases (oracle.py:80-174);
* ``paged``     -- the region-major page byte format, the slot store and the
                   block-table gather/dequant (layout.py:16-284, paged.py:30-91,
                   dequant.py:29-157);
* ``attention`` -- decode / MTP-verify attention with int8-quantized Q and the
                   kernel's masking rules (oracle.py:100-163,
                   native/xe2_kv_ops.cpp:657-791, :1086-1166) and chunked
                   prefill with fp Q and a bottom-right causal mask
                   (dequant.py:245-261, :448-501; onednn_prefill.py:89-121).

How each part is pinned (tests/test_oracle.py): known-answer vectors in
``tests/golden`` (ties, zero rows, constant rows, clamps, the reference's
geometry constants), closed forms (a single key returns its value row, equal
keys average the values), invariants (round-trip error bounds), and reduction
to a library routine (torch's scaled_dot_product_attention on the dequantized
tensors); tests/test_oracle.py holds each check.
"""
