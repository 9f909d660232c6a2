"""HIP graph capture of the projection stack: every replay must reproduce the eager launches
bit for bit (deterministic kernels, no memset nodes), with eager work between replays."""

import pytest
import torch

from tests.gpu_util import banner

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m", [1, 40, 300])
def test_stack_graph_replays_match_eager(cuda, m):
    from solution import kernels
    from solution.stack import ProjectionStack, Qwen2Shape

    banner("graph replay", m)
    shape = Qwen2Shape(hidden=256, inter=640, kv=64)
    st = ProjectionStack.synthetic(shape, 2, 300, torch.float16, cuda, seed_base=21)
    st.set_tokens([0, m])
    outs = lambda: [t[:m].clone() for t in (st.y_qkv, st.y_o, st.y_gu, st.y_d, st.dx_d,  # noqa
                                             st.dx_gu, st.dx_o, st.dx_qkv)] + \
        [st.per_layer[0][k].clone() for k in ("gb_q", "gb_v", "ga_q", "ga_v")]
    st.step()
    torch.cuda.synchronize()
    ref = outs()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st.step()
    other = st.per_layer[1]
    for rep in range(3):
        for t in (st.y_qkv, st.y_d, st.dx_qkv):
            t.zero_()
        # eager work between replays, on the same buffers' neighbours
        kernels.linear_fwd(st.x2[:m], [st.layers[1]["o"]])
        g.replay()
        torch.cuda.synchronize()
        got = outs()
        for i, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), f"replay {rep}, output {i}"
    assert other is st.per_layer[1]
