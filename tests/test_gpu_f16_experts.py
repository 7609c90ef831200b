"""F16 / BF16 / F32 expert tensors (the reference's fp16 expert mode, quant_kernels.py:1962-1964:
weights loaded with load_float_tensor(..., dtype=torch.float16), the forward an fp16 F.linear,
:2011).  The device holds them as fp16 (PGMOE_F16) in the 64-row tile layout; the decode
kernels take them as fp16 dot products, the grouped GEMMs as MFMA B operands with no
decode.

* the F16 relayout is the tile layout of the fp16 bytes, computed on the host;
* whole layers match the oracle (which holds the same fp16 values) in decode (M <= 8) and
  prefill, with the forward's own routing bit-exact: F16 experts, BF16 experts (rounded to
  fp16 at load), F32 gate / up beside an F16 down projection, an F16 shared expert;
* the dense FFN with F16 matrices;
* an fp16 down projection of more than 8192 inputs is refused at load (the decode down
  kernel that would take it holds whole super-blocks per lane)."""

import numpy as np
import pytest

import oracle
from gpu_helpers import build_pair, check_forward_routing, check_layer_output, log, sample_tokens
from pgmoe.synth import DenseSpec, LayerSpec, SyntheticDense, SyntheticLayer, random_blocks

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

F32, F16, BF16, Q8_0, Q6_K = 0, 1, 30, 8, 14

SPECS = {
    "f16": LayerSpec("f16", 2048, 32, 4, 768, (F16, F16, F16)),
    "bf16": LayerSpec("bf16", 1024, 16, 4, 512, (BF16, BF16, BF16)),
    "f32_f16": LayerSpec("f32_f16", 1024, 16, 2, 512, (F32, F32, F16)),
    "f16_shared": LayerSpec("f16_shared", 1024, 16, 4, 512, (F16, F16, F16), norm_topk=False, arch="qwen2moe",
                            shared_inter=1024, shared_qtypes=(F16, F16, F16), shared_gate=True),
}
_cache = {}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    _cache.clear()


def test_f16_relayout_is_the_tile_layout():
    from pgmoe import ops
    rows, cols, n = 100, 512, 2  # ragged rows: zero padding rows in the last 64-row group
    raw = random_blocks(np.random.default_rng(3), F16, n * rows, cols)
    got = ops.relayout(F16, torch.from_numpy(raw).cuda(), n, rows, cols).cpu().numpy()
    w = raw.view(np.uint16).reshape(n, rows, cols)
    ng, nb = (rows + 63) // 64, cols // 256
    stride = ng * nb * 32 * 1024
    exp = np.zeros((n, ng * 64, cols), np.uint16)
    exp[:, :rows] = w
    # tile (rg, b): chunk c of row r (16 bytes: weights 256 b + 8 c .. + 8) at
    # ((rg nb + b) 32 + c) 1024 + 16 r
    t = exp.reshape(n, ng, 64, nb, 32, 8).transpose(0, 1, 3, 4, 2, 5).reshape(n, -1)
    assert got.size == n * stride
    assert np.array_equal(got.reshape(n, stride), t.view(np.uint8).reshape(n, stride))


def _pair(name):
    if name not in _cache:
        _cache.clear()
        torch.cuda.empty_cache()
        _cache[name] = build_pair(SPECS[name], seed=0)
    return _cache[name]


@pytest.mark.parametrize("name,Ms", [("f16", (1, 2, 4, 8, 40, 600)), ("bf16", (1, 8, 300)),
                                     ("f32_f16", (1, 3, 64)), ("f16_shared", (1, 4, 8, 100))])
def test_float_expert_layer(name, Ms):
    lay, ol, mod = _pair(name)
    assert mod.down_exps.qtype == F16 and mod.gate_exps.plane is None
    for M in Ms:
        log(f"float experts {name} M={M}")
        x = lay.draw_x(M)
        out = mod(torch.from_numpy(x).to("cuda:0"))
        _, idx, w = ol.route(x)
        check_forward_routing(mod, M, idx, w)
        toks = sample_tokens(M, 16)
        ref = ol.forward_tokens(x, idx, w, tokens=toks)
        # decode: exact fp16 weights into fp32 dot products; prefill: fp16 MFMA operands
        stats = check_layer_output(out.cpu().numpy()[toks], ref, rel_l2=1e-4 if M <= 8 else 1e-3)
        log(f"  {name} M={M}: {stats}")
    mod.check_status(sync=True)


@pytest.mark.parametrize("M", [1, 8, 300])
def test_dense_f16(M):
    from pgmoe import HipDenseMLP
    sp = DenseSpec("dense_f16", 1024, 2816, (F16, F16, F16))
    lay = SyntheticDense(sp, seed=0)
    mod = HipDenseMLP.from_gguf(lay.gguf, lay.config, 0, torch.device("cuda", 0))
    log(f"dense f16 M={M}")
    x = lay.draw_x(M)
    got = mod(torch.from_numpy(x).to("cuda:0")).float().cpu().numpy().reshape(M, -1)
    mats = [(F16, *shp, np.ascontiguousarray(lay.tensor(f"ffn_{p}.weight")))
            for p, shp in (("gate", (2816, 1024)), ("up", (2816, 1024)), ("down", (1024, 2816)))]
    toks = sample_tokens(M, 16)
    check_layer_output(got[toks], oracle.dense_forward(x, *mats, tokens=toks))


def test_long_fp16_down_refused_at_load():
    from pgmoe import HipSparseMoEMLP
    spec = LayerSpec("f16_long", 512, 2, 1, 8448, (Q8_0, Q8_0, F16))
    lay = SyntheticLayer(spec, seed=0)
    with pytest.raises(NotImplementedError):
        HipSparseMoEMLP(lay.gguf, lay.config, 0, torch.device("cuda", 0))
