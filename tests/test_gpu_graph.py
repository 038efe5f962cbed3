"""The library's calls under HIP stream capture (torch.cuda.CUDAGraph), as a
serving loop would use them: capture one DiT layer's attention calls and
linear-layer product once, then replay the graph for every step.

The entry points only enqueue kernels on the caller's stream -- no
allocation, no memset, no host synchronisation, no pointer kept between
calls -- so a replay must give exactly the eager calls' result.  Captured
here: the self-attention with RoPE and no workspace (kd_fa_rope_run, whose
staged schedule is a sequence of K pre-pass + attention launches), the same
through the allocation-free kd_fa_dit_run_static (query/key RMSNorm, K in
the library's static array), the masked text cross-attention (kd_fa_run),
the unmasked cross-attention of a long prompt (the persistent kernel, four
query tiles per workgroup) and a Q8_0 linear layer through a workspace
(kd_mm_run: weight expansion + product).  The graph is replayed several times with eager work of the
program between the replays, the inputs are rewritten in place between
replays, and every replay is compared bitwise with the eager calls on the
same inputs."""
import numpy as np
import pytest
import torch

import kd_fa
import kd_mm
import kd_oracle_quant as oq
from fa_common import AXES, D, SCALE_FACTOR, THETA, randn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


class Layer:
    """Static inputs and outputs of one layer's calls, and the calls."""

    def __init__(self):
        B, H, T, Hp, Wp = 2, 8, 4, 16, 16
        self.L = L = T * Hp * Wp
        self.q = torch.empty((B, H, L, D), dtype=torch.bfloat16, device=DEV)
        self.k = torch.empty_like(self.q)
        self.v = torch.empty_like(self.q)
        self.kx = torch.empty((B, H, 100, D), dtype=torch.bfloat16, device=DEV)
        self.vx = torch.empty_like(self.kx)
        self.mask = torch.full((B, 1, L, 104), float("-inf"), dtype=torch.float16, device=DEV)
        # a long prompt's cross-attention: 2 x 16 heads x 32 query tiles of
        # 256 rows = 1,024 units, four per workgroup of the persistent kernel
        self.ql = torch.empty((B, 16, 8192, D), dtype=torch.bfloat16, device=DEV)
        self.kl = torch.empty((B, 16, 300, D), dtype=torch.bfloat16, device=DEV)
        self.vl = torch.empty_like(self.kl)
        self.mask[0, :, :, :77] = 0
        self.mask[1, :, :, :31] = 0
        table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
        self.rope = kd_fa.rope_table(torch.from_numpy(table).to(DEV))
        wq = (randn((D,), torch.float32, 21) * 0.3 + 1.0).to(DEV)
        wk = (randn((D,), torch.float32, 22) * 0.3 + 1.0).to(DEV)
        self.norm = kd_fa.qk_norm(wq, wk, 1e-6)
        # a Q8_0 linear layer 1,024 tokens x 512 -> 256 with bias
        rng = np.random.default_rng(23)
        w = (rng.standard_normal((256, 512)) * 0.05).astype(np.float32)
        self.wq8 = kd_mm.QuantWeight(torch.from_numpy(oq.quantize_q8_0(w)).to(DEV), kd_mm.TYPE_Q8_0, 512)
        self.x = torch.empty((L, 512), dtype=torch.float32, device=DEV)
        self.bias = torch.from_numpy((rng.standard_normal(256) * 0.1).astype(np.float32)).to(DEV)

    def outputs(self):
        B, H, L = 2, 8, self.L
        return {"self": torch.empty((B, L, H, D), device=DEV),
                "static": torch.empty((B, L, H, D), device=DEV),
                "cross": torch.empty((B, L, H, D), device=DEV),
                "long": torch.empty((B, 8192, 16, D), device=DEV),
                "linear": torch.empty((L, 256), device=DEV)}

    def fill(self, seed):
        for j, t in enumerate((self.q, self.k, self.v, self.kx, self.vx, self.ql, self.kl, self.vl)):
            t.copy_(randn(tuple(t.shape), torch.bfloat16, seed + j))
        self.x.copy_(randn(tuple(self.x.shape), torch.float32, seed + 9))

    def calls(self, out):
        """Descriptors and workspace for `out`, and the function that
        enqueues every call on the current stream."""
        s = 1.0 / D ** 0.5
        d_self = kd_fa.make_desc(self.q, self.k, self.v, None, out["self"], s)
        d_static = kd_fa.make_desc(self.q, self.k, self.v, None, out["static"], s)
        d_cross = kd_fa.make_desc(self.q, self.kx, self.vx, self.mask, out["cross"], s)
        d_long = kd_fa.make_desc(self.ql, self.kl, self.vl, None, out["long"], s)
        d_lin = kd_mm.make_desc(self.wq8, self.x, self.bias, out["linear"])
        ws = torch.empty(max(kd_mm.workspace_size(d_lin), 16), dtype=torch.uint8, device=DEV)

        def run():
            assert kd_fa.run_desc(d_self, self.rope) == kd_fa.OK
            assert kd_fa.run_static(d_static, self.rope, self.norm) == kd_fa.OK
            assert kd_fa.run_desc(d_cross) == kd_fa.OK
            assert kd_fa.run_desc(d_long) == kd_fa.OK
            assert kd_mm.run_desc(d_lin, ws) == 0

        return run, (d_self, d_static, d_cross, d_long, d_lin, ws)


def test_layer_calls_replay_bitwise():
    _need_gpu()
    _announce("graph capture: staged rope_run, dit_run_static, masked cross-attn, long-prompt cross-attn, q8_0 linear")
    # this shape fits one round of workgroups, where kd_fa_rope_run would be
    # one on-load launch: ROUTE_STAGED keeps its staged launch sequence
    with kd_fa.routing(kd_fa.ROUTE_STAGED):
        _replay_layer()


def _replay_layer():
    layer = Layer()
    eager_out, graph_out = layer.outputs(), layer.outputs()
    run_eager, keep_e = layer.calls(eager_out)
    run_graph, keep_g = layer.calls(graph_out)

    layer.fill(100)
    run_eager()          # also the library's once-per-device set-up, outside the capture
    run_graph()
    torch.cuda.synchronize()
    for name in eager_out:
        assert torch.equal(graph_out[name], eager_out[name]), name

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run_graph()
    torch.cuda.synchronize()

    other = torch.randn((512, 512), device=DEV)
    for rep, seed in enumerate((200, 200, 300, 400)):
        layer.fill(seed)
        for t in graph_out.values():
            t.fill_(float("nan"))
        run_eager()
        # the program's own work between the replays
        other = torch.tanh(other @ other.T * 1e-3)
        g.replay()
        torch.cuda.synchronize()
        for name in eager_out:
            assert torch.isfinite(eager_out[name]).all(), (rep, name)
            assert torch.equal(graph_out[name], eager_out[name]), (rep, name)
    del keep_e, keep_g
