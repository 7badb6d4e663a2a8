"""CPU restatement of the GPT speedrun rig's training-step hot path.

TEST INFRASTRUCTURE ONLY.  This package is the checker, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product path (``gptrig``) never imports,
calls or falls back to anything in here.

The reference (honglu2875/GPT-speedrun-TPU) is JAX 0.11 + Pallas-TPU and cannot
run in this image (Python 3.10, no jax).  Every function below restates one
reference function in torch-CPU (float32 arithmetic, bfloat16 rounding applied
where the reference casts), citing the reference file:line it follows.

Pinning (what keeps a mistake in this restatement from passing silently):

* attention fwd   - brute-force per-row softmax loops (tests/test_oracle_attention.py),
                    causal-prefix invariance, document independence,
                    single-segment equivalence, padding transparency; the
                    kernel-numerics forward: the exact float64 softmax when
                    its probabilities are left unrounded (every tile shape,
                    padding, block skipping, documents), the one-chunk closed
                    form with bf16 probabilities, the reference's tile choice.
* attention bwd   - float64 torch autograd of the dense softmax formula
                    (an independent derivation of the same gradient).
* FLCE fwd/bwd    - dense log-softmax + autograd; storage-row zero grads;
                    invalid targets -> +inf and zero grads; the reference
                    test inputs regenerated from numpy seeds 7/11/29.
* RoPE            - position 0 identity and norm preservation (the reference's
                    own test), closed-form rotation by pure Python trig.
* RMSNorm, GELU   - closed forms evaluated in float64 / pure Python.
* AdamW, LR       - hand-computed first steps, closed-form LR endpoints.
* init_params     - the reference's known parameter counts (116,160 smoke;
                    tier TPP denominators 59,918,208 ... 989,943,808).
* top-k routing   - brute force over all expert pairs on small inputs.

Bit-level agreement with XLA-CPU's fused bf16 elementwise code (where XLA's
excess-precision default decides whether an intermediate is rounded) cannot be
pinned without importing the reference: those points are tolerance-pinned and
documented as such in each function.
"""

from . import attention, flce, model, moe, nn, optim  # noqa: F401
