"""Greedy sampling on the GPU (ndl_greedy_argmax) against torch's argmax.

Reference: needle/model/sampler.py:27-28 (int(logit.argmax()) per greedy row).  The kernel
must return torch's index exactly: the first of equal maxima, a NaN above every number (the
first NaN), -0 equal to +0.  Cases: random rows of the real vocabulary (151,936), rows drawn
from a handful of values (ties everywhere, the common case of flat bf16 logits), NaN and
-inf rows, a vocabulary that is not a multiple of 8 read through a wider row stride, rows
that need an aligned copy first (an odd vocabulary, a shifted slice, a transposed view), every
dtype, int32 and int64 outputs, rows scanned in one slice or several (ties across a slice
edge), the workspace check, and the launches recorded in a HIP graph and replayed with eager
work in between.
"""
import pytest
import torch

from needle_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _want(logits):
    return logits.float().cpu().argmax(dim=-1)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,vocab", [(1, 151936), (48, 151936), (256, 151936), (3, 8),
                                        (5, 1000)])
def test_argmax_random_rows(dtype, rows, vocab):
    g = torch.Generator().manual_seed(rows * 7 + vocab)
    logits = (torch.randn(rows, vocab, generator=g) * 3).to(dtype).to(DEV)
    got = ops.greedy_argmax(logits)
    assert got.dtype == torch.int64
    assert torch.equal(got.cpu(), _want(logits))
    assert torch.equal(got.cpu(), logits.argmax(dim=-1).cpu())   # torch on the same GPU


@pytest.mark.parametrize("dtype", DTYPES)
def test_argmax_ties_take_the_first_index(dtype):
    g = torch.Generator().manual_seed(5)
    vals = torch.tensor([-2.0, -0.0, 0.0, 1.5, 3.0])
    logits = vals[torch.randint(0, 5, (64, 151936), generator=g)].to(dtype).to(DEV)
    logits[7] = 0.0
    logits[8] = -0.0
    logits[8, 50] = 0.0                                       # -0 and +0 tie: index 0
    logits[9] = -2.0
    logits[9, 151935] = 3.0                                   # the last entry
    out32 = torch.empty(64, dtype=torch.int32, device=DEV)
    got = ops.greedy_argmax(logits, out=out32)
    assert got is out32
    want = _want(logits)
    assert torch.equal(got.cpu().long(), want)
    assert want[7] == 0 and want[8] == 0 and want[9] == 151935


@pytest.mark.parametrize("dtype", DTYPES)
def test_argmax_nan_and_inf_rows(dtype):
    logits = torch.zeros(6, 4096, dtype=dtype, device=DEV)
    logits[0, 17] = float("nan")
    logits[0, 3000] = float("inf")                            # NaN beats +inf
    logits[1, 5] = float("nan")
    logits[1, 4] = float("nan")                               # the first NaN
    logits[2] = float("-inf")                                 # all -inf: index 0
    logits[3, 2000] = float("inf")
    logits[3, 1000] = float("inf")
    logits[4] = float("-inf")
    logits[4, 4095] = -1e4
    logits[5, 9] = float("nan")
    logits[5, 10] = float("inf")
    got = ops.greedy_argmax(logits).cpu()
    assert got.tolist() == [17, 4, 0, 1000, 4095, 9]
    assert torch.equal(got, logits.argmax(dim=-1).cpu())


def test_argmax_strided_rows_and_tail():
    g = torch.Generator().manual_seed(11)
    wide = torch.randn(9, 1008, generator=g).to(torch.bfloat16).to(DEV)
    wide[:, 1003] = 100.0                                     # outside the view: ignored
    view = wide[:, :1003]                                     # vocab % 8 == 3, stride 1008
    view[4, 1001] = 50.0                                      # inside the tail
    got = ops.greedy_argmax(view)
    assert torch.equal(got.cpu(), _want(view))
    assert got[4].item() == 1001


@pytest.mark.parametrize("dtype", DTYPES)
def test_argmax_unaligned_rows_are_copied_aligned(dtype):
    """Rows the kernel cannot read in place (a contiguous vocabulary of 50,257, not a multiple
    of 8; a column slice starting one element in; a transposed view) go through an aligned
    copy and still give torch's index."""
    g = torch.Generator().manual_seed(17)
    odd = (torch.randn(37, 50257, generator=g) * 3).to(dtype).to(DEV)
    odd[5, 50256] = 1000.0                                    # the last element of a row
    got = ops.greedy_argmax(odd)
    assert torch.equal(got.cpu(), _want(odd)) and got[5].item() == 50256
    base = (torch.randn(6, 1025, generator=g) * 3).to(dtype).to(DEV)
    shifted = base[:, 1:]                                     # data_ptr 2 or 4 bytes in
    assert torch.equal(ops.greedy_argmax(shifted).cpu(), _want(shifted))
    cols = (torch.randn(300, 7, generator=g) * 3).to(dtype).to(DEV).t()   # [7, 300], stride (1, 7)
    out = torch.empty(7, dtype=torch.int32, device=DEV)
    ops.greedy_argmax(cols, out=out)
    assert torch.equal(out.cpu().long(), _want(cols))


def test_argmax_in_a_graph():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(32, 151936, generator=g).to(torch.bfloat16).to(DEV)
    out = torch.zeros(32, dtype=torch.int32, device=DEV)
    ops.greedy_argmax(logits, out=out)                        # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.greedy_argmax(logits, out=out)
    for i in range(4):
        logits.copy_(torch.randn(32, 151936, generator=g).to(torch.bfloat16))
        out.fill_(-1)                                         # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.cpu().long(), _want(logits)), f"replay {i}"


def test_argmax_rejects_bad_arguments():
    from needle_amd._lib import NeedleAmdError
    with pytest.raises((ValueError, NeedleAmdError)):          # not [rows, vocab]
        ops.greedy_argmax(torch.zeros(2, 4, 104, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(TypeError):
        ops.greedy_argmax(torch.zeros(4, 104, dtype=torch.int32, device=DEV))
    with pytest.raises(ValueError):
        ops.greedy_argmax(torch.zeros(4, 104, dtype=torch.bfloat16, device=DEV),
                          out=torch.zeros(3, dtype=torch.int64, device=DEV))
    assert ops.greedy_argmax(torch.zeros(0, 104, dtype=torch.bfloat16, device=DEV)).numel() == 0


@pytest.mark.parametrize("rows,vocab", [(1, 600000), (3, 151936), (600, 151936), (2, 8200),
                                        (17, 16384)])
def test_argmax_slices(rows, vocab):
    """One slice per row (many rows), several (few rows, long rows, up to the 64-slice cap),
    slices ending inside the last 8-element chunk."""
    from needle_amd import _lib
    g = torch.Generator().manual_seed(rows + vocab)
    logits = torch.randn(rows, vocab, generator=g).to(torch.bfloat16).to(DEV)
    logits[0, vocab - 1] = 50.0                               # the very last entry
    if rows > 1:
        logits[1, 8191] = 60.0                                # at a slice edge
        logits[1, 8192] = 60.0                                # tie across it: the first wins
    got = ops.greedy_argmax(logits)
    assert torch.equal(got.cpu(), _want(logits))
    lib = _lib.load()
    print(f"rows {rows} vocab {vocab}: workspace "
          f"{lib.ndl_greedy_argmax_workspace_bytes(rows, vocab)} bytes")


def test_argmax_workspace_too_small_is_refused():
    import ctypes
    from needle_amd import _lib
    lib = _lib.load()
    logits = torch.zeros(2, 151936, dtype=torch.bfloat16, device=DEV)
    out = torch.zeros(2, dtype=torch.int64, device=DEV)
    need = lib.ndl_greedy_argmax_workspace_bytes(2, 151936)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    rc = lib.ndl_greedy_argmax(out.data_ptr(), 1, logits.data_ptr(), 151936, 2, 151936,
                               _lib.NDL_DTYPE_BF16, ws.data_ptr(), need - 8, st)
    assert rc == -3                                           # NDL_ERR_WORKSPACE
    rc = lib.ndl_greedy_argmax(out.data_ptr(), 1, logits.data_ptr(), 151936, 2, 151936,
                               _lib.NDL_DTYPE_BF16, None, 0, st)
    assert rc == -3
    rc = lib.ndl_greedy_argmax(out.data_ptr(), 1, logits.data_ptr(), 151936, 2, 151936,
                               _lib.NDL_DTYPE_BF16, ws.data_ptr(), need, st)
    assert rc == 0
    torch.cuda.synchronize()
    assert out.tolist() == [0, 0]
