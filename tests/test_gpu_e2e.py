"""GPU: a complete SiHC sublayer denoiser routed by the HIP ops.

Pattern of the reference's integration test (research/tests/test_sublayer_kernels.py:
216-263, full model vs a literal dense carrier): the same model, same weights and
same inputs, once with the HIP ops and once with the oracle's PyTorch read/write
(run on the same device), compared on the output and on every parameter gradient.
"""
from __future__ import annotations

import copy

import pytest
import torch

from helpers import announce, assert_close_reference, assert_parity, rel_l2
from oracle import sihc_oracle as O
from sihc_hip.e2e import SiHCDenoiser

pytestmark = pytest.mark.gpu


def _oracle_routing(model):
    model.read = lambda x, alpha: O.read(x, alpha)
    model.triangular = lambda base, ups, gamma: O.triangular_torch(base, ups, gamma)
    model.write = lambda x, ups, beta: O.write(x, ups, beta)
    return model


def _small(schedule, depth=8, patch=8, seed=0):
    stages = (8,) if depth == 8 else (8, 12)
    torch.manual_seed(seed)
    return SiHCDenoiser(hidden=64, depth=depth, heads=4, patch=patch, stages=stages,
                        schedule=schedule).random_init(seed=seed).cuda()


def _inputs(batch=2, seed=1):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(batch, 3, 256, 256, device="cuda", generator=g)
    t = torch.rand(batch, device="cuda", generator=g)
    y = torch.randint(0, 1000, (batch,), device="cuda", generator=g)
    return x, t, y


@pytest.mark.parametrize("depth,patch", [(8, 8), (20, 8), (8, 4)])
def test_stage_schedule_model_matches_oracle_routing_fp32(depth, patch):
    announce(f"e2e stage fp32 depth={depth} patch={patch}")
    model = _small("stage", depth, patch)
    ref = _oracle_routing(copy.deepcopy(model))
    x, t, y = _inputs()
    out, expected = model(x, t, y), ref(x, t, y)
    out.float().square().mean().backward()
    expected.float().square().mean().backward()
    assert_parity(out, expected, torch.float32, what="output")
    for (name, a), (_, b) in zip(model.named_parameters(), ref.named_parameters()):
        assert a.grad is not None and torch.isfinite(a.grad).all(), name
        # gradients pass through attention/MLP bodies: compare in relative L2
        assert rel_l2(a.grad, b.grad) < 1e-4, (name, rel_l2(a.grad, b.grad))


def test_literal_schedule_model_matches_stage_schedule_fp32():
    announce("e2e literal vs stage fp32")
    lit = _small("literal")
    stage = _oracle_routing(copy.deepcopy(lit))
    stage.schedule = "stage"
    x, t, y = _inputs()
    a, b = lit(x, t, y), stage(x, t, y)
    a.float().square().mean().backward()
    b.float().square().mean().backward()
    assert rel_l2(a, b) < 1e-5
    for (name, p), (_, q) in zip(lit.named_parameters(), stage.named_parameters()):
        assert rel_l2(p.grad, q.grad) < 1e-4, (name, rel_l2(p.grad, q.grad))


def test_bf16_model_matches_oracle_routing():
    announce("e2e stage bf16")
    model = _small("stage").to(torch.bfloat16)
    ref = _oracle_routing(copy.deepcopy(model))
    x, t, y = _inputs()
    with torch.no_grad():
        out, expected = model(x.bfloat16(), t, y), ref(x.bfloat16(), t, y)
    assert_parity(out, expected, torch.bfloat16, what="bf16 output", kind="chained")


AUTOCAST_CASES = [(s, d, p) for s in ("stage", "literal") for d, p in ((8, 4), (12, 8), (20, 4))]


@pytest.mark.parametrize("schedule,depth,patch", AUTOCAST_CASES,
                         ids=[f"{s}-d{d}-p{p}" for s, d, p in AUTOCAST_CASES])
def test_bf16_autocast_training_step_matches_oracle_routing(schedule, depth, patch):
    # The training path the reference runs (fp32 parameters under bf16 autocast,
    # sihc/training/train.py:633-639), output and every parameter gradient against the same
    # model routed by the oracle's PyTorch read/write, with the reference's tolerances for
    # this comparison (research/tests/test_sublayer_kernels.py:247-266: output by
    # assert_numerics, gradients atol 5e-4 / rtol 0.15). Depth 8, 12 and 20 (stages 8,
    # 12 and 8 + 12) with 4- and 16-slot cells (patch 8 and 4).
    announce(f"e2e bf16 autocast {schedule} depth={depth} patch={patch}: output and all gradients")
    stages = {8: (8,), 12: (12,), 20: (8, 12)}[depth]
    torch.manual_seed(19)
    model = SiHCDenoiser(hidden=64, depth=depth, heads=4, patch=patch, stages=stages,
                         schedule=schedule).random_init(seed=19).cuda()
    ref = _oracle_routing(copy.deepcopy(model))
    ref.event = lambda x, dz, beta, alpha: O.event_forward(x, dz, beta, alpha)
    x, t, y = _inputs(batch=1, seed=7)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = model(x, t, y)
        expected = ref(x, t, y)
    assert out.dtype == torch.bfloat16
    out.float().square().mean().backward()
    expected.float().square().mean().backward()
    assert_parity(out, expected, torch.bfloat16, what="autocast output", kind="chained")
    assert_close_reference(out, expected, atol=0.025, rtol=0.03, what="autocast output")
    for (name, a), (_, b) in zip(model.named_parameters(), ref.named_parameters()):
        assert a.grad is not None and b.grad is not None, name
        assert torch.isfinite(a.grad).all(), name
        assert_close_reference(a.grad, b.grad, atol=5e-4, rtol=0.15, what=f"grad {name}")


@pytest.mark.parametrize("schedule", ["stage", "literal"])
def test_xl_denoiser_cfg_batch_matches_oracle_routing(schedule):
    # Benchmark config 4 at its size: the SiHC-XL sublayer denoiser (D = 1152, 28 blocks,
    # 16 heads, stages 8/12/8) in bf16, batch 64 class-conditional + 64 unconditional, routed
    # once by the HIP ops and once by the oracle's PyTorch read/write on the same device
    # (pattern of the reference's research/tests/test_sublayer_kernels.py:245-258).
    announce(f"e2e XL config 4 batch 128 schedule={schedule} vs oracle routing")
    model = SiHCDenoiser(schedule=schedule).random_init(seed=4).cuda().to(torch.bfloat16).eval()
    ref = _oracle_routing(copy.deepcopy(model))
    ref.event = lambda x, dz, beta, alpha: O.event_forward(x, dz, beta, alpha)
    g = torch.Generator(device="cuda").manual_seed(40)
    x = torch.randn(128, 3, 256, 256, device="cuda", generator=g).to(torch.bfloat16)
    t = torch.rand(128, device="cuda", generator=g)
    y = torch.cat([torch.randint(0, 1000, (64,), device="cuda", generator=g),
                   torch.full((64,), 1000, device="cuda")])
    with torch.no_grad():
        out = model(x, t, y)
        expected = ref(x, t, y)
    assert out.shape == (128, 3, 256, 256) and torch.isfinite(out.float()).all()
    # 56 routing events deep, each carrier rounded on both sides: a chain
    assert_parity(out, expected, torch.bfloat16, what=f"XL {schedule} output (batch 128)", kind="chained")


def _ctx(schedule, seed=0, depth=8):
    torch.manual_seed(seed)
    stages = (8,) if depth == 8 else (8, 12)
    return SiHCDenoiser(hidden=64, depth=depth, heads=4, patch=8, stages=stages, schedule=schedule,
                        in_context_len=4, in_context_start=2).random_init(seed=seed).cuda()


@pytest.mark.parametrize("schedule", ["stage", "literal"])
def test_in_context_model_matches_oracle_routing_fp32(schedule):
    # SublayerSiHCInContextModel behaviour (sublayer.py:84-128): prefix tokens join the
    # workspace sequence from block 2 on and never enter the routing.
    announce(f"e2e in-context {schedule} fp32")
    model = _ctx(schedule, depth=20)
    ref = _oracle_routing(copy.deepcopy(model))
    ref.schedule = "stage"  # the oracle routes the same recurrence late-materialised
    x, t, y = _inputs()
    out, expected = model(x, t, y), ref(x, t, y)
    out.float().square().mean().backward()
    expected.float().square().mean().backward()
    assert rel_l2(out, expected) < 1e-5
    for (name, a), (_, b) in zip(model.named_parameters(), ref.named_parameters()):
        assert a.grad is not None and torch.isfinite(a.grad).all(), name
        assert rel_l2(a.grad, b.grad) < 1e-4, (name, rel_l2(a.grad, b.grad))
    assert model.in_context_posemb.grad.abs().sum() > 0


@pytest.mark.parametrize("schedule", ["stage", "literal"])
def test_whole_model_fullgraph_compile(schedule):
    # The whole denoiser (bodies + HIP routing ops) traced without a graph break; the
    # routing ops run through their fake implementations at trace time.
    announce(f"e2e fullgraph compile {schedule}")
    torch._dynamo.reset()
    model = _ctx(schedule)
    twin = copy.deepcopy(model)
    x, t, y = _inputs()
    eager = model(x, t, y)
    eager.float().square().mean().backward()
    compiled = torch.compile(twin, backend="aot_eager", fullgraph=True)
    out = compiled(x, t, y)
    out.float().square().mean().backward()
    assert rel_l2(out, eager) < 1e-6
    for (name, a), (_, b) in zip(twin.named_parameters(), model.named_parameters()):
        assert rel_l2(a.grad, b.grad) < 1e-5, (name, rel_l2(a.grad, b.grad))


def test_model_forward_hip_graph_replay():
    # Inference forward captured once and replayed on new inputs (the reference's
    # CUDA-graph sampling path, sampling.py:6-11), with eager work between replays.
    announce("e2e hip graph forward")
    model = _ctx("literal").to(torch.bfloat16).eval()
    x, t, y = _inputs()
    sx, st, sy = x.bfloat16().clone(), t.clone(), y.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.no_grad(), torch.cuda.stream(side):
        for _ in range(2):
            model(sx, st, sy)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(graph):
        static_out = model(sx, st, sy)
    for r in range(3):
        nx, nt, ny = _inputs(seed=10 + r)
        sx.copy_(nx.bfloat16())
        st.copy_(nt)
        sy.copy_(ny)
        graph.replay()
        with torch.no_grad():
            expected = model(nx.bfloat16(), nt, ny)
        torch.cuda.synchronize()
        assert torch.equal(static_out, expected), f"replay {r} differs from eager"


def test_checkpoint_round_trip(tmp_path):
    # state_dict -> file -> weights-only load into a fresh model: identical outputs.
    # The connection parameters keep the reference's names and layout
    # (blocks.{i}.{attention,mlp}_connection.{read,write}_weight, [D, S] fp32).
    announce("e2e checkpoint round trip")
    model = _ctx("stage", seed=3)
    path = tmp_path / "ckpt.pt"
    torch.save(model.state_dict(), path)
    fresh = SiHCDenoiser(hidden=64, depth=8, heads=4, patch=8, stages=(8,), in_context_len=4,
                         in_context_start=2).cuda()
    fresh.load_state_dict(torch.load(path, weights_only=True))
    x, t, y = _inputs()
    with torch.no_grad():
        assert torch.equal(model(x, t, y), fresh(x, t, y))
    keys = set(fresh.state_dict())
    for i in range(8):
        for conn in ("attention_connection", "mlp_connection"):
            for w in ("read_weight", "write_weight"):
                k = f"blocks.{i}.{conn}.{w}"
                assert k in keys and fresh.state_dict()[k].shape == (64, 4) and fresh.state_dict()[k].dtype == torch.float32
