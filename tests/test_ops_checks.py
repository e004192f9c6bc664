"""Argument checks of the Python operator layer (webyiq_amd/ops.py), on the
CPU: the C ABI receives raw device pointers, so the wrapper rejects what the
kernels would silently misread (int64 token ids read as pairs of uint32,
non-contiguous views, short outputs) before anything is launched.  CPU
tensors pass every check but the last (a cuda device), so each rejection
below is the one under test."""
import numpy as np
import pytest
import torch

from webyiq_amd import ops

K, G = 256, 128


def weight(rows=64):
    return ops.Q4Tensor(torch.zeros((rows, K // 8), dtype=torch.int32), torch.zeros((rows, K // G), dtype=torch.int32),
                        K, G)


def acts(M=2, GA=None):
    return ops.empty_acts(M, K, GA, G, device="cpu")


def test_int64_ids_rejected():
    w = weight()
    with pytest.raises(ValueError, match="tok: dtype torch.int64"):
        ops.embed(w, torch.arange(3))
    with pytest.raises(ValueError, match="ids: dtype torch.int64"):
        ops.gather_rows(w, torch.arange(3))
    with pytest.raises(ValueError, match="ids: dtype torch.int64"):
        ops.argmax(torch.zeros((2, 64)), ids=torch.arange(64))
    with pytest.raises(ValueError, match="ids: dtype torch.int64"):
        ops.lm_head_argmax(w, acts(), ids=torch.arange(64), workspace=torch.zeros(1 << 14, dtype=torch.uint8))


def test_short_outputs_rejected():
    w = weight()
    a = acts(M=2)
    with pytest.raises(ValueError, match="y: shape"):
        ops.gemv(w, a, mode=ops.MODE_ACCUMULATE, y=torch.zeros((2, 63)))
    with pytest.raises(ValueError, match="y: shape"):
        ops.gemm(w, a, y=torch.zeros((1, 64)))
    with pytest.raises(ValueError, match="out: shape"):
        ops.lm_head_argmax(w, a, out=torch.zeros(1, dtype=torch.int32),
                           workspace=torch.zeros(1 << 14, dtype=torch.uint8))
    with pytest.raises(ValueError, match="logits: shape"):
        ops.lm_head_argmax(w, a, logits=torch.zeros((2, 32)), workspace=torch.zeros(1 << 14, dtype=torch.uint8))
    with pytest.raises(ValueError, match="workspace: .* at least"):
        ops.lm_head_argmax(w, a, workspace=torch.zeros(8, dtype=torch.uint8))
    with pytest.raises(ValueError, match="ids: .* at least 64"):
        ops.lm_head_argmax(w, a, ids=torch.zeros(10, dtype=torch.int32),
                           workspace=torch.zeros(1 << 14, dtype=torch.uint8))
    with pytest.raises(ValueError, match="out: shape"):
        ops.embed(w, torch.zeros(3, dtype=torch.int32), out=torch.zeros((3, K - 4)))


def test_layout_and_dtype_rejected():
    w = weight()
    x = torch.zeros((2, 2 * K))[:, ::2]  # non-contiguous view
    with pytest.raises(ValueError, match="x: not contiguous"):
        ops.quant(x)
    with pytest.raises(ValueError, match="x: dtype torch.float64"):
        ops.quant(torch.zeros((2, K), dtype=torch.float64))
    with pytest.raises(ValueError, match="w.q: shape"):
        ops.gemv(ops.Q4Tensor(w.q[:, :8].contiguous(), w.s, K, G), acts())
    with pytest.raises(ValueError, match="acts.xq: dtype torch.uint8"):
        ops.gemv(w, ops.Acts(torch.zeros((2, K), dtype=torch.uint8), torch.zeros((2, 1)),
                             torch.zeros((2, 2), dtype=torch.int32), K, G))
    with pytest.raises(ValueError, match="acts.xs: shape"):
        ops.gemv(w, ops.Acts(torch.zeros((2, K), dtype=torch.int8), torch.zeros((2, 1)),
                             torch.zeros((2, 1), dtype=torch.int32), K, G))
    with pytest.raises(ValueError, match="do not match the weight"):
        ops.gemv(ops.Q4Tensor(torch.zeros((64, 64), dtype=torch.int32), torch.zeros((64, 4), dtype=torch.int32),
                              512, G), acts())
    with pytest.raises(ValueError, match="norm: shape"):
        ops.quant(torch.zeros((2, K)), norm=torch.ones(K - 1))


def test_valid_cpu_arguments_stop_at_the_device_check():
    """Everything else valid: the only complaint left is the CPU device."""
    w = weight()
    with pytest.raises(ValueError, match="expected a cuda tensor"):
        ops.gemv(w, acts())
    with pytest.raises(ValueError, match="expected a cuda tensor"):
        ops.embed(w, torch.zeros(3, dtype=torch.int32))
    with pytest.raises(ValueError, match="expected a cuda tensor"):
        ops.quant(torch.from_numpy(np.zeros((2, K), np.float32)))
