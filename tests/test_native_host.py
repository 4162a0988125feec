"""Host logic of the in-process native front end (no GPU): engine lookup order (reference native.py:18-22) and the
ChatML turn text (qwen_vk.cpp:615-620)."""
import os
from pathlib import Path

import pytest

from seedplane_amd import native


def test_find_engine_order(tmp_path, monkeypatch):
    a, b, c = tmp_path / 'a.so', tmp_path / 'b.so', tmp_path / 'c.so'
    for p in (a, b, c):
        p.write_bytes(b'')
    monkeypatch.setattr(native, 'REPO_ENGINE', c)
    monkeypatch.setenv('SEEDPLANE_NATIVE_ENGINE', str(b))
    assert native.find_engine(str(a)) == str(a)          # explicit first
    assert native.find_engine() == str(b)                # then the environment
    monkeypatch.delenv('SEEDPLANE_NATIVE_ENGINE')
    assert native.find_engine() == str(c)                # then the in-repo build
    assert native.find_engine(str(tmp_path / 'missing.so')) == str(c)   # a missing explicit path falls through


def test_find_engine_missing(tmp_path, monkeypatch):
    monkeypatch.setattr(native, 'REPO_ENGINE', tmp_path / 'none.so')
    monkeypatch.delenv('SEEDPLANE_NATIVE_ENGINE', raising=False)
    monkeypatch.setattr(native.ctypes.util, 'find_library', lambda name: None)
    with pytest.raises(FileNotFoundError):
        native.find_engine()


def test_chat_turn_template():
    first = native.chat_turn([], 'SYS', 'hi')
    assert first == '<|im_start|>system\nSYS<|im_end|>\n<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n'
    # an assistant reply that ended on <|im_end|> (id 7) is not closed again
    assert native.chat_turn([1, 7], 'SYS', 'x', im_end_id=7) == '\n<|im_start|>user\nx<|im_end|>\n<|im_start|>assistant\n'
    # a reply cut by the token budget is closed first
    assert native.chat_turn([1, 2], 'SYS', 'x', im_end_id=7) == ('<|im_end|>\n<|im_start|>user\nx<|im_end|>\n'
                                                                  '<|im_start|>assistant\n')


def test_bad_mode_is_rejected_before_loading(tmp_path):
    with pytest.raises(ValueError):
        native.NativeEngine(tmp_path, mode='bogus')
