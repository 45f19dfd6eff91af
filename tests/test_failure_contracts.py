"""The reference's failure contracts on the serving side, checked on the host (no GPU needed):
the errors a caller written against the reference catches are the ones raised here."""

from __future__ import annotations

import types

import pytest
import torch

from kv_skill_v2_amd.decode_reader import DecodeReader, DecodeReaderDeviceError, DecodeReaderError
from kv_skill_v2_amd.pool import LibraryPool


def test_decode_reader_errors_are_assertion_errors():
    """DecodeReader's precondition errors are ValueError (this build) and AssertionError (the
    reference asserts them, xenc/d23_read_kernels.py:146-150)."""
    assert issubclass(DecodeReaderError, ValueError) and issubclass(DecodeReaderError, AssertionError)
    assert issubclass(DecodeReaderDeviceError, RuntimeError) and issubclass(DecodeReaderDeviceError, AssertionError)
    with pytest.raises(AssertionError):
        DecodeReader(4, 36, 4, 64, 128, "cpu")        # 9 query heads per kv head
    with pytest.raises(ValueError):
        DecodeReader(4, 16, 4, 60, 128, "cpu")        # head dim not a multiple of 8
    with pytest.raises(AssertionError):
        DecodeReader(4, 16, 4, 64, 128, "cpu")        # no CPU path: the reference asserts q.is_cuda


def test_full_pool_raises_out_of_memory():
    """A full LibraryPool raises torch.cuda.OutOfMemoryError, as the reference's static pool does
    (xenc/d23_vllm_plugin.py:181-183), and leaves its free list unchanged."""
    pool = types.SimpleNamespace(free=[(0, 3), (7, 2)])
    with pytest.raises(torch.cuda.OutOfMemoryError):
        LibraryPool._alloc(pool, 4)
    assert pool.free == [(0, 3), (7, 2)]
    assert LibraryPool._alloc(pool, 2) == 0 and pool.free == [(2, 1), (7, 2)]   # first fit
