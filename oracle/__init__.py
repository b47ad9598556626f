"""CPU oracle for the Qwen3.6 MoE decode layer and Gated DeltaNet step.

TEST INFRASTRUCTURE ONLY.  This package restates, on the CPU, the maths of
the reference's PyTorch oracle (suryavanshi/fastkernels,
src/fastkernels/reference/*.py) so the HIP kernels can be checked against it.
Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may
import it, and only as the checker / the timed CPU baseline: the product
(fastkernels_amd) never imports, calls or falls back to anything here.

Floating-point work is restated with torch CPU ops in fp32 (the reference
upcasts every operand with `.float()`); the integer routing tables
(histogram, offsets, stable permutation) are restated in numpy.

Pinning (what checks each function against something other than itself):
  rms_norm            closed-form KAT of tests/test_qwen36_spec.py:368-377
  router top-k        brute-force ranking at E<=16, exact-tie cases, torch.topk
                      on untied inputs, sum-to-one invariant
  expert_histogram    numpy.bincount / collections.Counter
  moe_align           invariants (stable sort by expert, counts == histogram,
                      perm o inverse == id, offsets == exclusive cumsum) and a
                      brute-force sort at small sizes
  expert MLP / MoE    float64 dense restatement (all experts, one-hot gates),
                      fixed-routing fixture [3,17,42,89,127,199,231,255]
  causal conv         torch.nn.functional.conv1d (library routine) and the
                      unit-tap closed form y = silu(x)
  gated delta rule    closed forms: S=0 gives o = beta * v * (k . q); decay
                      with A_log=-inf is 1; T-token call == T one-token calls;
                      float64 brute force at Hk=2, Hv=4, D=8
  gated RMSNorm       closed form on a constant vector
  synthetic blocks    float64 brute force at the tiny spec
  rope                position 0 is the identity; pair norms kept; the two
                      pairings are one dim permutation apart; complex-number
                      restatement; dot products depend on the offset only
  attention           torch scaled_dot_product_attention (library routine)
                      with expanded kv heads and an offset causal mask; one
                      position gives the value row; cache rows outside the
                      step untouched
  synthetic attention float64 restatement with RoPE as complex
                      multiplication and torch scaled_dot_product_attention
                      over expanded kv heads; caller's caches untouched, rows
                      other than the step's unchanged
No function is left "parity unpinned" at the north-star tolerances; the only
unpinned behaviours are torch.topk's tie order (replaced here by the
documented lower-id rule) and cross-version bf16 rounding of the synthetic
bf16 oracle.
"""

from .qwen36 import *  # noqa: F401,F403
from .qwen36 import __all__  # noqa: F401
