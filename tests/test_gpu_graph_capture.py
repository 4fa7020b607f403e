"""The loss, forward and backward, captured into a HIP graph.

The C ABI enqueues everything on the caller's stream and neither synchronises
the host nor allocates device memory (the module allocates its buffers with
torch.empty, which graph capture serves from the graph's pool), so a training
step that calls the loss can be captured whole.  The graph is replayed several
times, with eager work and synchronisations between the replays, and every
replay is checked against the eager result.
"""
import pytest
import torch

from helpers import max_rel, randn_pair, rel_err
from memoryefficientclip_amd import MemoryEfficientCLIPLoss, MemoryEfficientLiTLoss

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skip(reason="the first case ended in a host segmentation fault inside torch.cuda.graph's "
                            "capture_end (stream-capture end / graph instantiation) on the MI355X box; the cause "
                            "is not identified, so the test stays off the GPU; the module refuses capture "
                            "with a RuntimeError (tests/test_api_cpu.py::test_graph_capture_is_refused) and every "
                            "C-ABI entry point with MEC_ERR_UNSUPPORTED "
                            "(tests/test_abi_cpu.py::test_graph_capture_is_refused_before_any_launch)"),
]
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("lit", [False, True], ids=["clip", "lit"])
def test_fwd_bwd_under_graph_capture(dtype, lit):
    n, d = 2300, 128
    a, b = randn_pair(n, d, seed=41, dtype=dtype)
    ga = a.to(DEV).requires_grad_(True)
    gb = b.to(DEV).requires_grad_(not lit)
    mod = MemoryEfficientLiTLoss(0.07) if lit else MemoryEfficientCLIPLoss(0.07)
    say(f"graph capture {dtype} {'LiT' if lit else 'CLIP'} n={n} d={d}")

    # eager reference
    loss = mod(ga, gb)
    loss.backward()
    ref = (loss.detach().clone(), ga.grad.clone(), None if lit else gb.grad.clone())

    # warm-up on a side stream (as graph capture requires), then capture one step
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            ga.grad = None
            gb.grad = None
            mod(ga, gb).backward()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    ga.grad = None
    gb.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_loss = mod(ga, gb)
        static_loss.backward()
    torch.cuda.synchronize()

    for rep in range(3):
        # unrelated eager work on the same buffers' device between replays
        junk = torch.randn(1 << 20, device=DEV)
        (junk * 2).sum().item()
        graph.replay()
        torch.cuda.synchronize()
        el = rel_err(static_loss.detach().cpu(), ref[0].cpu())
        ea = max_rel(ga.grad.cpu(), ref[1].cpu())
        eb = 0.0 if lit else max_rel(gb.grad.cpu(), ref[2].cpu())
        say(f"  replay {rep}: loss rel {el:.2e}, grads {ea:.2e} {eb:.2e}")
        # the forward sums use relaxed atomics, so replays may differ in the last bits
        assert el < 1e-6 and ea < 1e-5 and eb < 1e-5
