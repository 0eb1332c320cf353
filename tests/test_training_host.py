"""Host-side pieces of the training path that are plain PyTorch compositions
(no HIP call), checked on the CPU in float64 against the modules they stand in
for: the per-edge Linear with the split-K weight gradient (values, forces-style
first differentiation with create_graph=True, and the second differentiation to
the inputs and parameters, including a first differentiation that skips the
weight gradient), the split-K product with rows left over, and run_seq over a
RadialProfile net (on the CPU every LayerNorm + SiLU pair runs as the modules)."""
import torch

from ubio_molfm_amd import modules
from ubio_molfm_amd import second_order as so


def _rel(a, b):
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


def test_splitk_matches_plain_product():
    g = torch.Generator().manual_seed(1)
    for E in (5, 2048 * 3, 2048 * 32 + 7, 2048 * 40 + 1):
        a = torch.randn(E, 9, generator=g, dtype=torch.float64)
        b = torch.randn(E, 5, generator=g, dtype=torch.float64)
        assert _rel(so._splitk_tn(a, b), a.t() @ b) < 1e-13, E


def test_edge_linear_second_order_matches_linear():
    torch.manual_seed(0)
    E, k, n = 2048 * 4 + 37, 24, 16
    lin = torch.nn.Linear(k, n).double()
    p = torch.randn(E, k, dtype=torch.float64, requires_grad=True)
    R = torch.randn(E, k, dtype=torch.float64)

    def run(f):
        x = torch.sin(p) * 1.3
        y = f(x)
        e = (torch.tanh(y) ** 2).sum()
        gp, = torch.autograd.grad(e, p, create_graph=True)     # the weight gradient is not asked for
        L = (gp * R).sum() + e
        return [y, gp] + list(torch.autograd.grad(L, [p, lin.weight, lin.bias]))

    got = run(lambda x: so.edge_linear(lin, x))
    ref = run(lin)
    for a, b in zip(got, ref):
        assert _rel(a, b) < 1e-12


def test_run_seq_matches_radial_profile_on_cpu():
    torch.manual_seed(2)
    prof = modules.RadialProfile([32, 64, 64, 16]).double()
    h = torch.randn(300, 64, dtype=torch.float64)
    assert not so.ln_silu_fusable(prof.net[1], h)
    assert torch.equal(so.run_seq(prof.net[1:], h), prof.net[1:](h))
