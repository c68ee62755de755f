"""Host logic of ``kernels.linear.SumSq`` (no GPU): which tensor a buffer of row sums describes,
so that a norm never takes sums written for other rows. The device side (what the sums hold and
the norms' outputs with them) is tests/test_gpu_sumsq.py."""

import torch

from kernels.linear import SumSq


def written(ss, y):
    buf = ss._out(y)
    ss._wrote(y)
    return buf


def test_sums_describe_only_the_tensor_written():
    ss = SumSq()
    y = torch.zeros((5, 4096), dtype=torch.bfloat16)
    buf = written(ss, y)
    assert buf.dtype == torch.float32 and buf.numel() >= 5 * 4096 // 16
    assert ss._of(y) is buf
    assert ss._of(y.view(5, 4096)) is buf  # a view of the same rows
    assert ss._of(y.clone()) is None  # another tensor
    assert ss._of(y[:4]) is None  # other rows
    assert ss._of(y[1:]) is None  # another address
    assert ss._of(y.view(10, 2048)) is None  # another shape


def test_an_in_place_change_retires_the_sums():
    ss = SumSq()
    y = torch.zeros((8, 1024), dtype=torch.bfloat16)
    written(ss, y)
    y.add_(1)
    assert ss._of(y) is None


def test_the_next_producer_retires_the_previous_sums():
    ss = SumSq()
    y = torch.zeros((8, 1024), dtype=torch.bfloat16)
    z = torch.zeros((8, 1024), dtype=torch.bfloat16)
    written(ss, y)
    ss._out(z)  # a producer started (its launch may still fail): y's sums no longer count
    assert ss._of(y) is None and ss._of(z) is None
    ss._wrote(z)
    assert ss._of(z) is not None and ss._of(y) is None


def test_the_written_storage_stays_alive_while_described():
    ss = SumSq()
    y = torch.zeros((8, 1024), dtype=torch.bfloat16)
    ptr = y.data_ptr()
    written(ss, y)
    del y
    # the storage is held, so no new tensor can take its address and pass for the old rows
    fresh = [torch.zeros((8, 1024), dtype=torch.bfloat16) for _ in range(8)]
    assert all(t.data_ptr() != ptr for t in fresh)


def test_the_buffer_grows_and_keeps_its_address_otherwise():
    ss = SumSq()
    small = written(ss, torch.zeros((2, 512), dtype=torch.bfloat16))
    again = written(ss, torch.zeros((4, 1024), dtype=torch.bfloat16))
    assert again.data_ptr() == small.data_ptr()  # 4 x 64 parts fit the first buffer
    big = written(ss, torch.zeros((16, 65536), dtype=torch.bfloat16))
    assert big.numel() >= 16 * 4096
