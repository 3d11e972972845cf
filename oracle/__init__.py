"""oracle — a CPU restatement of decision.js's scoring path, used ONLY as the checker.

This package is test infrastructure. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
may import it, and only to check or time against; the product (decision.js_amd/) never imports it and has
no CPU fallback.

  ref.py    numpy restatement of every kernel and engine step, with the reference's f16 storage points
            (each function cites the reference file:line it follows)
  c/        plain-C restatement of the integer/byte parts (f16 rounding, q8/q4 dequantization, quantize8,
            forest packing), built by oracle/Makefile into oracle/_build/liboracle.so

Pinning (what checks each function; see tests/test_oracle.py):
  dequant, gather            brute force over all codes x all 65,536 f16 scales against the C restatement
                             and the closed form RNE(code x scale)
  quantize8                  closed form; round trip; C restatement
  quantize4                  golden vectors written by tests/golden/make_q4_golden.py from the reference's
                             own export_common.quantize4
  packing (forest, prefix,   brute-force masks of kernels.ts:135 / d3-kernels.ts:223 / eg2 ranges; position
  encoder)                   and leaf invariants; C restatement
  rmsnorm, rope, attention,  float64 textbook forms (rotation as a complex product, softmax(QK^T)V with an
  glu, leaf logits, pool     explicit mask), closed-form special cases
  decoder forward            shared-trunk == unshared sequences (causal invariant), float64 re-run
There is no runnable reference here (WGSL needs a WebGPU runtime; the reference's Python needs the network),
so the forward pass itself has no reference golden vectors: its parity rests on the checks above.
"""
