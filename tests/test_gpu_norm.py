"""GPU parity of pgmoe_add_rmsnorm (exec_fused_add_rmsnorm / exec_fused_rmsnorm /
GGUFRMSNorm drop-ins) against the CPU oracle: h and the normalised output bit for bit
(the kernel and the oracle share one summation order), over row widths that take each
kernel variant, input dtypes fp32 / fp16 / bf16, and fp16 / fp32 outputs; then the norm
feeding the MoE block as at model.py:1037-1039."""

import numpy as np
import pytest

import oracle
from gpu_helpers import build_pair, check_layer_output, log
from pgmoe.synth import CONFIGS

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)


def _bits(a):
    return a.view(np.uint16 if a.dtype == np.float16 else np.uint32)


@pytest.mark.parametrize("R,D", [(1, 2048), (3, 256), (4096, 2048), (7, 3584), (2, 4096), (5, 8192), (3, 14336),
                                 (2, 100), (0, 512)])
@pytest.mark.parametrize("xdt,ddt", [("f32", "f32"), ("f32", "f16"), ("f16", None), ("bf16", "bf16")])
def test_add_rmsnorm_bitexact(dev, R, D, xdt, ddt):
    from pgmoe import exec_fused_add_rmsnorm, exec_fused_rmsnorm
    log(f"add_rmsnorm R={R} D={D} x={xdt} delta={ddt}")
    rng = np.random.default_rng(R * 31 + D)
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
    x = torch.from_numpy(rng.standard_normal((R, D)).astype(np.float32) * 3).to(tdt[xdt])
    d = None if ddt is None else torch.from_numpy(rng.standard_normal((R, D)).astype(np.float32)).to(tdt[ddt])
    w = torch.from_numpy((rng.standard_normal(D) * 0.5 + 1.0).astype(np.float32))

    def host(t):  # numpy view the oracle takes (bf16 as uint16 bits)
        if t is None:
            return None
        return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()

    bf = (xdt == "bf16", ddt == "bf16")
    for odt, ondt in ((torch.float16, np.float16), (torch.float32, np.float32)):
        if d is not None:
            h, out = exec_fused_add_rmsnorm(x.to(dev), d.to(dev), w.to(dev), 1e-6, out_dtype=odt)
        else:
            h, out = None, exec_fused_rmsnorm(x.to(dev), w.to(dev), 1e-6, out_dtype=odt)
        rh, rout = oracle.add_rmsnorm(host(x), host(d), w.numpy(), 1e-6, out_dtype=ondt, bf16=bf)
        assert out.dtype == odt and out.shape == (R, D)
        assert np.array_equal(_bits(out.cpu().numpy()), _bits(rout))
        if h is not None:
            assert h.dtype == torch.float32
            assert np.array_equal(_bits(h.cpu().numpy()), _bits(rh))


def test_module_and_errors(dev):
    from pgmoe import GGUFRMSNorm
    w = torch.linspace(0.5, 1.5, 1024)
    norm = GGUFRMSNorm(w.to(dev), 1e-5)
    x = torch.randn(1, 6, 1024, device=dev)
    d = torch.randn(1, 6, 1024, device=dev)
    h, y = norm.forward_with_residual(x, d)
    assert h.shape == x.shape and y.dtype == torch.float16
    assert torch.equal(h, x + d)
    y2 = norm(x + d, out_dtype=torch.float16)
    assert torch.equal(y, y2)
    assert norm(x).dtype == torch.float32  # out_dtype None: the input's dtype
    with pytest.raises(NotImplementedError):
        norm(x, out_dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        norm.forward_with_residual(x, d[:, :3])


def test_norm_feeds_the_moe_block(dev):
    """h, normed = ffn_norm.forward_with_residual(x, attn_delta); out = h + mlp(normed)
    (model.py:1037-1042) with the HIP norm and MoE block, against the oracle's chain, at the
    Qwen3-30B-A3B decode shape (M = 1 and 4) and a prefill M = 64."""
    from pgmoe import GGUFRMSNorm
    lay, ol, mod = build_pair(CONFIGS["qwen3_30b_a3b"], seed=0)
    H = mod.hidden
    rng = np.random.default_rng(9)
    w = (rng.standard_normal(H) * 0.1 + 1.0).astype(np.float32)
    norm = GGUFRMSNorm(torch.from_numpy(w).to(dev), 1e-6)
    for M in (1, 4, 64):
        log(f"norm -> moe M={M}")
        x = (rng.standard_normal((M, H)) * 2).astype(np.float32)
        delta = rng.standard_normal((M, H)).astype(np.float32)
        h, normed = norm.forward_with_residual(torch.from_numpy(x).to(dev).view(1, M, H),
                                               torch.from_numpy(delta).to(dev).view(1, M, H))
        out = (h + mod(normed).float()).view(M, H).cpu().numpy()
        rh, rn = oracle.add_rmsnorm(x, delta, w, 1e-6)
        assert np.array_equal(normed.view(M, H).cpu().numpy().view(np.uint16), rn.view(np.uint16))
        _, idx, tw = ol.route(rn)
        toks = np.arange(M) if M <= 8 else np.array([0, 17, M - 1])
        ref = rh[toks].astype(np.float64) + ol.forward_tokens(rn, idx, tw, tokens=toks)
        check_layer_output(out[toks], ref)
