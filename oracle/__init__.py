"""CPU restatement of bux's MoE expert path, in numpy: the checker of this repository's
HIP kernels. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may
import this package, and only to check or to time the CPU path beside the GPU one. The
product (``bux_amd``) never imports it and has no CPU fallback.

Modules:

- `oracle.mxfp8`: the MXFP8 1x32 quantizer, bit for bit as
  ``src/bux/architecture/precision/blockscaled.py:282-356`` computes it, and its
  dequantization (``:223-229``);
- `oracle.moe`: the token path (``src/bux/architecture/experts/moe.py:776-1066``), the
  grouped GEMMs off a Blackwell GPU (``grouped_blockscaled.py:92-317``,
  ``grouped.py:42-102``), the ragged tile list (``grouped_mxfp8.py:157-182``), the
  expert activation (``layers/mlp.py:20-35``, ``common/functional.py:12-40``) and the
  MoE layer's forward and backward composed from them;
- `oracle.router`: the router's forward (``src/bux/architecture/experts/moe.py:236-284,
  474-483``): logits, scores, group limit, top-k, weights;
- `oracle.bf16`: bfloat16 as uint16 bits, rounding to nearest even.

What pins each function (golden vectors, exhaustive checks, closed forms, brute force)
is listed in each module's header; ``tests/test_oracle.py`` runs those pins.
"""
