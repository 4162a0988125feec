"""seedplane_amd: MI355X (gfx950) implementation of SeedPlane's Qwen2 decode step and speculative verification.

Modules mirror the reference package: `qwen_engine` (Qwen2Engine, KVCache, chat_prompt), `speculative` (forest,
verify_greedy, ledger, batched tree verification), `native` (NativeEngine-compatible in-process front end).  The
compute runs in libseedplane_hip.so (seedplane_amd/csrc, C ABI in include/seedplane_hip.h).
"""
__all__ = ['qwen_engine', 'speculative', 'native']
