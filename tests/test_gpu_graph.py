"""HIP graph capture of the DiT loop.

Every entry point on the step's path launches its kernels on the caller's stream and allocates
nothing itself (torch allocates the outputs), and no launch records a memset, so the whole loop can
be captured into one HIP graph, the serving loop's way to remove per-launch gaps. Two blocks at the
single-block shape (1x30x52 = 1560 tokens, 512 text tokens) are captured with ``torch.cuda.graph``;
the graph is replayed three times with the program's own eager work and synchronizations between
the replays, and every replay must equal the eager forward bit for bit (on the step's shape a graph
replay was measured at 1013.7 ms against 1014.7-1015.8 ms eager).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

GRID = (1, 30, 52)
S, DIM, NBLK = 1560, 5120, 2


def test_dit_forward_graph_replays_match_eager(pkg, dev):
    blk = pkg.block
    g = torch.Generator(device=dev).manual_seed(99)
    blocks = [blk.random_block_weights(dev, g, qk_gamma_mean=1.0, keep_raw=False)[0] for _ in range(NBLK)]
    h0 = torch.randn(S, DIM, device=dev, generator=g).to(torch.bfloat16)
    temb = torch.randn(6, DIM, device=dev, generator=g)
    ctx = torch.randn(512, DIM, device=dev, generator=g).to(torch.bfloat16)
    rope = pkg.rope_tables(GRID, device=dev)
    crosses = [blk.project_cross_kv(w, ctx) for w in blocks]
    tables = torch.stack([w.scale_shift_table for w in blocks])
    eager = blk.dit_forward(blocks, h0, temb, rope, crosses, tables=tables)
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on a side stream before capture, as torch requires
        blk.dit_forward(blocks, h0, temb, rope, crosses, tables=tables)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = blk.dit_forward(blocks, h0, temb, rope, crosses, tables=tables)
    torch.cuda.synchronize()

    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from the eager forward"
        again = blk.dit_forward(blocks, h0, temb, rope, crosses, tables=tables)
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
