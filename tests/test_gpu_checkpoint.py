"""A packed checkpoint loaded onto the GPU runs through the HIP kernels and agrees with the host."""

from __future__ import annotations

import pytest
import torch

from llmopt.quantization import QuantLinear, load_quantized_, quantize_model_, save_quantized
from tests.test_checkpoint_host import TinyBlock

pytestmark = pytest.mark.gpu


def test_checkpoint_runs_on_gpu(tmp_path):
    model = quantize_model_(TinyBlock(0).to(torch.bfloat16), bits=4, group_size=128, symmetric=False)
    ids = torch.randint(0, 32, (2, 9), generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        ref = model(ids)
    save_quantized(model, tmp_path / "ckpt")
    gpu = load_quantized_(TinyBlock(7).to(torch.bfloat16), tmp_path / "ckpt").to("cuda")
    assert isinstance(gpu.up, QuantLinear) and gpu.up.qweight.is_cuda
    with torch.no_grad():
        out = gpu(ids.to("cuda")).float().cpu()
    err = float((out - ref.float()).abs().max() / ref.float().abs().max())
    assert err <= 1e-2
