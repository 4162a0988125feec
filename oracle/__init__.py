"""ORACLE -- test infrastructure, not product code.

CPU restatements of the reference's algorithms on the decode / speculative-verify path, used only as the checker by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.  Nothing in seedplane_amd imports this package.

  qwen_ref.py         Qwen2Engine forward/generate in fp32 (seedplane/qwen_engine.py), with the sliding-window
                      and tree-ancestor masks, quantized weights dequantized once at load.
  quant_ref.py        closed-form dequantisation of the int8 block-32 and int4 group-32 formats.
  speculative_ref.py  forest / verify_greedy / ledger (seedplane/speculative.py), the linear batched verify with
                      rollback (experiments/hive_scaling/benchmark_speculative.py:59-135), and the float64
                      acceptance-sampling rule (speculative sampling with residual max(p - q, 0)).

How each part is pinned (checks in tests/test_oracle_*.py):
  * forward: against transformers' Qwen2ForCausalLM on the reference's tiny fixture (the reference established
    Qwen2Engine == Transformers to 2.29e-5, experiments/v17/RESULTS.md:12-13), position invariance
    (tests/test_core.py:168-175), window >= context == full attention, HF sliding-window masking rule, tree-masked
    logits == linear causal logits of each root path.
  * RMSNorm / RoPE: closed forms (constant vector, pair-norm preservation, relative-position property).
  * dequant: hand-worked codes, nibble order, round trip of the packer layout.
  * verify_greedy / forest / ledger: the reference's own unit tests (tests/test_speculative.py:14-44).
  * acceptance sampling: exact enumeration on tiny vocabularies (output distribution == p, the speculative
    sampling theorem) and reduction to greedy verification as T -> 0.
"""
