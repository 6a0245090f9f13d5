"""The kernel-level binding example of INTEGRATION.md agrees with the library's prototypes
(CPU: the block loads the library and sets argtypes; nothing is called on a device)."""

import ctypes

import torch

from integration_example import load_example
from recap_amd import _lib


def test_example_prototypes_match_the_abi():
    ns = load_example()
    lib = ns["lib"]
    for name in ("recap_kv_pack", "recap_block_sparse_attn"):
        got = list(getattr(lib, name).argtypes)
        want = list(_lib.SIGNATURES[name][1])
        assert got == want, name
    assert lib.recap_last_error.restype is ctypes.c_char_p
    assert ns["DTYPE"] == {torch.float16: _lib.RECAP_F16, torch.bfloat16: _lib.RECAP_BF16}
    assert callable(ns["block_sparse_exact"])
