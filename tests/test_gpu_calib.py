"""The streaming-read calibration kernel (logo_read_calibration) on the GPU:
with ordinary and with non-temporal loads, over sizes that are not a multiple
of the grid's stride and at the grid limits, it reads the buffer without
writing anything (the sink keeps its contents unless a workgroup's XOR of its
words equals the sentinel, which a buffer of bf16 ones never gives: every
lane folds an even number of equal words)."""

import pytest
import torch

from logo_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,grid", [(16, 1), (4096 * 16 + 48, 3), (1 << 24, 65536), ((1 << 24) + 16, 257)])
@pytest.mark.parametrize("nontemporal", [0, 1])
def test_calibration_reads_without_writing(gpu, nbytes, grid, nontemporal):
    lib = _lib.lib()
    buf = torch.ones(nbytes // 2, dtype=torch.bfloat16, device=gpu)
    sink = torch.full((grid,), 7, dtype=torch.int32, device=gpu)
    print(f"calibration nbytes={nbytes} grid={grid} nt={nontemporal}", flush=True)
    _lib.check(lib.logo_read_calibration(_lib.ptr(buf), nbytes, _lib.ptr(sink), grid, nontemporal,
                                         _lib.stream_of(buf)), "logo_read_calibration")
    torch.cuda.synchronize()
    assert bool((sink == 7).all())
    assert bool((buf == 1).all())
