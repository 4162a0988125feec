"""The reference's import path for the decode / verification path: `seedplane.<module>` is `seedplane_amd.<module>`
(the same module object), so callers and tests written against the reference package -- `from
seedplane.speculative import SpeculativeForest, verify_greedy, CommitLedger`, `from seedplane.qwen_engine import
Qwen2Engine, chat_prompt` -- run on this build unchanged.  Provided: qwen_engine, speculative, engine, native,
native_bundle.  The reference package's other modules (planner, llama backend, hive transport, CLI) lie outside this
path and are not provided."""
