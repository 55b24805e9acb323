"""The launch guard makes the tensors' device current only when it is not already (CPU-only checks)."""

import contextlib

import torch

from popcorn_amd import _lib


def test_no_switch_on_the_current_device(monkeypatch):
    monkeypatch.setattr(_lib, "_get_device", lambda: 0)
    assert isinstance(_lib.on_device(torch.device("cuda", 0)), contextlib.nullcontext)
    assert isinstance(_lib.on_device(torch.device("cuda")), contextlib.nullcontext)  # no index: current


def test_switch_to_another_device(monkeypatch):
    monkeypatch.setattr(_lib, "_get_device", lambda: 0)
    guard = _lib.on_device(torch.device("cuda", 1))
    assert isinstance(guard, torch.cuda.device) and guard.idx == 1  # entered only around the launch
