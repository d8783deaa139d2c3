"""CPU oracle for the batched multi-LoRA INT4 linear: TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on its fast path's fused linear layer, so the HIP
library can be checked against it. Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`
may import it, and only as the checker (or, in `bench.py`, as the timed CPU baseline). Nothing in `jeff_amd/` imports
it; the product path fails loudly when the HIP library is missing and never falls back to this code.

Modules (each function cites the reference file:line it restates; paths are relative to the reference checkout):
- `bf16`:    float32 -> bfloat16 round-to-nearest-even on the bit pattern, and back.
- `codec`:   the on-disk nibble codec and the kernel's word layout (`engine/int4.py:183-262`), the dequantisation
             `bf16((c - z) * s)` (`engine/int4.py:203-208`, `engine/int4_kernels.py:57-59`), g64 or g128, zeros.
- `routing`: adapter id per request row -> stable segment sort (replaces `adp[t // row_len]`,
             `engine/fast_path.py:167,189`).
- `readout`: the decision head, per-adapter readout logits rounded to bfloat16 and the masked, tempered softmax
             (`engine/batched_kernels.py:492-559`).
- `epilogue`: residual add + RMSNorm and SiLU(gate) * up around the linear (`engine/fast_path.py:80-156,295-298`).
- `layer`:   the reference's torch layer `LoraLinear.forward` applied per adapter segment (`engine/lora.py:204-220`)
             in "model" and "float32" precision; the float64 exact result and the forward error bounds of
             `tests/test_int4_kernels_cuda.py:108-168`.

How each function is pinned (checked by `tests/test_oracle_*.py` against golden vectors, closed forms and brute force):
- bf16 RNE: against torch's own float32->bfloat16 conversion on every tie pattern and random bits, and against an
  exact rational rounding (fractions) on a sample.
- codec: the reference's golden words (0xFED98710, 0x88888888 padding, low-nibble-first bytes) from
  `tests/test_int4.py:211-264`, round trips, and jeff-asic's packing restated in `tests/test_int4.py:221-229`.
- dequant: the reference's special case 7 x 1.0078125 (`tests/test_int4.py:312-317`), brute force over every code,
  every zero point and every finite positive bfloat16 scale against float64 products rounded by exact rationals.
- routing: invariants (bijection, stable order, one adapter per segment, coverage) and equality with
  `adp[t // row_len]` on uniform rows, brute force on tiny inputs.
- layer: the float64 exact result against an independent per-element sum; the bound model is the reference's own.
- epilogue: x + d bit for bit against torch's float32 addition; the norm against the reference's standard-path
  formula in torch float32 (`rms`, `engine/fast_path.py:295-298`) and closed forms (a constant row, a zero row), planted
  mistakes (no eps, a mean over n - 1, no w1); SiLU against torch's float64 silu and its limits.
- readout: logits against a per-element sum in exact rationals on small inputs (and so the rounding through float32
  to bfloat16 on every value), planted mistakes (another adapter's readout, a transposed readout); the softmax against
  closed forms (one option kept gives 1, equal logits give 1/count, a temperature t equals logits divided by t at
  temperature 1), torch's float32 softmax, and the reference's mask value -1e9.
"""
