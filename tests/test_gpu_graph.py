"""The no-grad (prefill / evaluation) chain forward captured in a HIP graph: every library launch takes its
addresses and sizes by value and allocates nothing, and torch's allocations come from the graph's pool, so the
whole pass replays without host work. Replays are checked bitwise against eager passes, with eager work and
synchronization between them, and after the inputs' contents change (the graph reads its static inputs)."""
import pytest
import torch

from gpu_helpers import DEV

pytestmark = pytest.mark.gpu


def _chain_forward(cell, h0, D, K, mode):
    stack = cell.new_stack(h0.shape, h0.dtype, h0.device, mode=mode)
    h, deltas, keys, coeffs, prior = h0, [], [], None, None
    for s in range(len(D)):
        l, blk = divmod(s, K)
        hs = h + D[s]
        deltas.append(stack.write(s, hs, h) if stack is not None else hs - h)
        h, coeffs, prior = cell.combine(hs, h0, deltas, coeffs, prior, l, blk, keys=keys, stack=stack)
    return h


@pytest.mark.parametrize("mode", ["scores", "stack", "list"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_forward_chain_replays_in_a_graph(mode, dtype):
    from loopback_amd.cell import LoopDeltaAttnRes
    K, R, d, t = 2, 4, 256, 300
    gen = torch.Generator().manual_seed(5)
    cell = LoopDeltaAttnRes(d, R, K).to(DEV)
    with torch.no_grad():
        cell.query.copy_((torch.randn(K * R - 1, d, generator=gen) * 0.5).to(DEV))
    h0 = torch.randn(2, t, d, generator=gen).to(dtype).to(DEV)
    D = [torch.randn(2, t, d, generator=gen).to(dtype).to(DEV) for _ in range(K * R)]
    print(f"case graph {mode} {dtype}", flush=True)
    with torch.no_grad():
        ref = _chain_forward(cell, h0, D, K, mode).clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            _chain_forward(cell, h0, D, K, mode)                    # warm-up on a side stream
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = _chain_forward(cell, h0, D, K, mode)
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
            eager = _chain_forward(cell, h0, D, K, mode)           # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(eager, ref)
        D[3].mul_(-0.5)
        h0.add_(0.25)
        ref2 = _chain_forward(cell, h0, D, K, mode).clone()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref2) and not torch.equal(ref2, ref)


@pytest.mark.parametrize("mode", ["scores", "stack", "list"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_training_chain_replays_in_graphs(mode, dtype):
    """The chain's forward and backward captured as one HIP graph (chain.capture_training): every replay -- with eager
    chains and synchronizations between them, and after the inputs' contents change -- gives the eager pass's final
    state, loss and every gradient (h0, each update, the query) bitwise."""
    from loopback_amd.chain import ChainConfig, capture_training, make_inputs, run_chain
    cfg = ChainConfig(f"graph-train-{mode}", 256, 2, 4, 2, 300, dtype, True, q_std=0.5)
    h0, D, Q, G = make_inputs(cfg, DEV)
    print(f"case graph training {mode} {dtype}", flush=True)

    def eager():
        h, loss, g = run_chain(cfg, h0, D, Q, G, mode)
        torch.cuda.synchronize()
        return h.clone(), loss.clone(), [g["h0"].clone(), g["query"].clone()] + [x.clone() for x in g["D"]]

    ref = eager()
    step = capture_training(cfg, h0, D, Q, G, mode)
    for k in range(4):
        h, loss, g = step()
        torch.cuda.synchronize()
        got = [g["h0"].clone(), g["query"].clone()] + [x.clone() for x in g["D"]]
        assert torch.equal(h, ref[0]) and torch.equal(loss, ref[1]), k
        assert all(torch.equal(a, b) for a, b in zip(got, ref[2])), k
        again = eager()                                   # eager work between replays
        assert torch.equal(again[0], ref[0])
    with torch.no_grad():
        D[5].mul_(-0.5)
        h0.add_(0.25)
    ref2 = eager()
    h, loss, g = step()
    torch.cuda.synchronize()
    assert torch.equal(h, ref2[0]) and torch.equal(loss, ref2[1]) and not torch.equal(ref2[0], ref[0])
    got = [g["h0"].clone(), g["query"].clone()] + [x.clone() for x in g["D"]]
    assert all(torch.equal(a, b) for a, b in zip(got, ref2[2]))


def test_training_pass_replays_at_config3():
    """Config 3 whole (d=1024, K=3, R=4, 16384 tokens, bf16, fwd+bwd), the pass as one graph: three replays with an
    eager pass between each give the eager pass's final state, loss and every gradient bitwise."""
    from loopback_amd.chain import CONFIGS, capture_training, make_cell, make_inputs, run_chain
    cfg = CONFIGS["c3"]
    h0, D, Q, G = make_inputs(cfg, DEV)
    cell = make_cell(cfg, Q)
    print("case graph training config 3", flush=True)

    def eager():
        h, loss, g = run_chain(cfg, h0, D, Q, G, "scores", cell=cell)
        torch.cuda.synchronize()
        return [h.clone(), loss.clone(), g["h0"].clone(), g["query"].clone()] + [x.clone() for x in g["D"]]

    ref = eager()
    step = capture_training(cfg, h0, D, Q, G, "scores")
    for k in range(3):
        h, loss, g = step()
        torch.cuda.synchronize()
        got = [h, loss, g["h0"], g["query"]] + list(g["D"])
        assert all(torch.equal(a, b) for a, b in zip(got, ref)), k
        assert torch.equal(eager()[0], ref[0])
