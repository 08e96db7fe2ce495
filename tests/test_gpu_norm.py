"""GPU parity of the fused residual add + RMSNorm of the step loop.

The reference's ops (engine/mamba.py:82-89 RMSNorm after the residual add
of Mamba.step's layer loop) run by torch on the same GPU are the reference.
x + add is the same fp32 addition (bit-identical); the normalised rows sum
the squares in another order, so they compare to 1e-6 norm-wise.
"""

import pytest
import torch

from redpanda_amd.norm import hip_add_rmsnorm

pytestmark = pytest.mark.gpu
dev = "cuda"


def rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def nrel(a, b):
    return float((a - b).abs().max() / (b.abs().max() + 1e-30))


@pytest.mark.parametrize("dt", [None, torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("R,d", [(4096, 512), (7, 768), (33, 100), (5, 1), (0, 64), (3, 1500)])
def test_add_rmsnorm_matches_torch(gpu_lib, R, d, dt):
    g = torch.Generator(device=dev).manual_seed(R + d)
    x = torch.randn(R, d, device=dev, generator=g) * 3
    w = 1 + 0.2 * torch.randn(d, device=dev, generator=g)
    add = None if dt is None else torch.randn(R, 2 * d, device=dev, generator=g).to(dt)[:, :d]
    xn, out = hip_add_rmsnorm(x, add, w, 1e-5)
    xr = x if add is None else x + add
    ref = rms(xr, w, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(xn, xr)
    if R:
        assert nrel(out, ref) <= 1e-6


def test_model_inference_step_uses_fused_norm(gpu_lib):
    """No-grad Mamba.step (fused add + norm) against the grad-mode step
    (torch's add and RMSNorm) on the same model and inputs."""
    from redpanda_amd import mamba as hm
    torch.manual_seed(0)
    m = hm.Mamba(hm.MambaConfig(d_model=256, n_layer=4, d_state=20, n_track_state=4,
                                vocab_size=64)).to(dev)
    emb = torch.randn(3, 64, 256, device=dev)
    with torch.no_grad():
        c1, o1 = None, []
        for t in range(3):
            h, c1 = m.step(input_embed=emb[t], cache=c1)
            o1.append(h)
    c2, o2 = None, []
    for t in range(3):
        h, c2 = m.step(input_embed=emb[t], cache=c2)  # records autograd: torch's ops
        o2.append(h.detach())
    torch.cuda.synchronize()
    for a, b in zip(o1, o2):
        assert nrel(a, b) <= 1e-6
