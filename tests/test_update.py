"""Gate-threshold budget controller (logo_amd/update.py against the behaviour
of logo/update.py:17-75), on the CPU: per-layer sign steps, untouched layers
without observations, cleared counters, argument checks, and the
two-process gloo case where every rank must apply the step of the summed
counts."""

import os
import socket

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

from logo_amd.layers import LoGoAttention, LoGoConfig
from logo_amd.update import update_gate_thres


def _model(layers=3, dtype=torch.float32):
    cfg = LoGoConfig(hidden_size=64, num_attention_heads=2, num_hidden_layers=layers)
    return torch.nn.ModuleList([LoGoAttention(cfg, i) for i in range(layers)]).to(dtype)


def _set(model, counts):
    for m, (g, t) in zip(model, counts):
        m.global_token_count.fill_(g)
        m.total_token_count.fill_(t)
        m.gate_avg.fill_(0.5 * t)


def test_sign_steps_and_reset():
    model = _model()
    _set(model, [(30, 100), (70, 100), (0, 0)])
    ratio = update_gate_thres(model, target_global_ratio=0.5, update_rate=0.01)
    assert ratio.shape == (3, 1)
    assert torch.allclose(ratio[:, 0], torch.tensor([0.3, 0.7, 0.0]))
    # ratio below target lowers the threshold (more tokens go global), above raises it
    assert [round(m.gate_thres.item(), 6) for m in model] == [0.49, 0.51, 0.5]
    for m in model:
        assert m.global_token_count.item() == 0 and m.total_token_count.item() == 0 and m.gate_avg.item() == 0


def test_exact_target_and_zero_rate():
    model = _model(2)
    _set(model, [(50, 100), (10, 100)])
    update_gate_thres(model, target_global_ratio=0.5, update_rate=0.0)
    assert [m.gate_thres.item() for m in model] == [0.5, 0.5]
    _set(model, [(50, 100), (10, 100)])
    update_gate_thres(model, target_global_ratio=0.5, update_rate=0.25)
    assert [m.gate_thres.item() for m in model] == [0.5, 0.25]


def test_bf16_threshold_steps_in_its_own_dtype():
    """After model.to(bf16) the threshold is bf16 (logo/layers/logo.py:73): the
    default 5e-4 step is below half an ulp at 0.5 and leaves it unchanged, as
    the reference's bf16 add_ does; a step of one ulp moves it."""
    model = _model(1, torch.bfloat16)
    assert model[0].gate_thres.dtype == torch.bfloat16 and model[0].total_token_count.dtype == torch.float32
    _set(model, [(90, 100)])
    update_gate_thres(model, target_global_ratio=0.5, update_rate=0.0005)
    assert model[0].gate_thres.item() == 0.5
    _set(model, [(90, 100)])
    update_gate_thres(model, target_global_ratio=0.5, update_rate=2 ** -8)
    assert model[0].gate_thres.item() == 0.5 + 2 ** -8


def test_argument_checks_and_no_layers():
    model = _model(1)
    with pytest.raises(ValueError):
        update_gate_thres(model, target_global_ratio=1.5)
    with pytest.raises(ValueError):
        update_gate_thres(model, update_rate=-1.0)
    assert update_gate_thres(torch.nn.Linear(2, 2)) is None


def _free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _worker(rank, world, port, out):
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        model = _model(2)
        # rank 0 sees 10 of 100 global tokens in layer 0, rank 1 sees 80 of 100:
        # summed 90 / 200 < 0.5 -> lower; layer 1: 60/100 + 60/100 -> raise
        _set(model, [(10 if rank == 0 else 80, 100), (60, 100)])
        ratio = update_gate_thres(model, target_global_ratio=0.5, update_rate=0.01)
        out[rank] = [ratio[0, 0].item(), ratio[1, 0].item(), model[0].gate_thres.item(), model[1].gate_thres.item()]
    finally:
        dist.destroy_process_group()


def test_two_ranks_gloo_share_one_step():
    port = _free_port()
    with mp.Manager() as mgr:
        out = mgr.dict()
        mp.spawn(_worker, args=(2, port, out), nprocs=2, join=True)
        res = dict(out)
    for rank in (0, 1):
        r0, r1, t0, t1 = res[rank]
        assert abs(r0 - 0.45) < 1e-6 and abs(r1 - 0.6) < 1e-6
        assert abs(t0 - 0.49) < 1e-6 and abs(t1 - 0.51) < 1e-6


@pytest.mark.gpu
def test_controller_after_gpu_training_steps(gpu):
    """Counters accumulated by LoGoAttention's training forward on the HIP
    path feed the controller, which steps the device threshold in place."""
    cfg = LoGoConfig(hidden_size=256, num_attention_heads=2, num_hidden_layers=1, gate_thres_init=0.5)
    layer = LoGoAttention(cfg).to(device=gpu, dtype=torch.bfloat16).train()
    g = torch.Generator()
    g.manual_seed(11)
    h = torch.randn(2, 300, 256, generator=g).bfloat16().to(gpu)
    with torch.no_grad():
        sel = (torch.sigmoid(layer.gate_proj(h)) >= layer.gate_thres).sum().item()
        layer(h)
        layer(h)
    assert layer.global_token_count.item() == 2 * sel and layer.total_token_count.item() == 1200
    ratio = update_gate_thres(layer, target_global_ratio=1.0, update_rate=2 ** -6)
    assert abs(ratio.item() - sel / 600) < 1e-6
    assert layer.gate_thres.item() == 0.5 - 2 ** -6 and layer.total_token_count.item() == 0
