"""Q4_0 / Q4_1 / Q5_0 experts on the GPU: the relayout of Q4_0 (Q5_0) bytes gives exactly
the device buffer of the Q4_1 (Q8_0) bytes with the same values, and whole layers with
Q4_0 experts (the format of the reference's synthetic qwen35moe test model), Q4_1 and Q5_0
experts match the oracle (rel-L2 <= 1e-3, max|d|/max|ref| <= 2e-2), decode and prefill."""

import numpy as np
import pytest

import oracle
from gpu_helpers import check_layer_output, log, sample_tokens
from pgmoe.synth import LayerSpec, SyntheticLayer, random_blocks
from test_q4_0_cpu import q4_0_as_q4_1, q5_0_as_q8_0

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
Q4_0, Q4_1, Q5_0, Q8_0, Q6_K = 2, 3, 6, 8, 14


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.mark.parametrize("qt", [Q4_0, Q5_0])
def test_q4_0_relayout_is_the_q8_0_layout_of_the_same_values(qt):
    from pgmoe import ops
    rng = np.random.default_rng(11)
    rows, cols, n = 100, 512, 3  # ragged row count: padded tile rows
    raw = random_blocks(rng, qt, n * rows, cols)
    conv, dt = (q4_0_as_q4_1, Q4_1) if qt == Q4_0 else (q5_0_as_q8_0, Q8_0)
    assert ops.device_qtype(qt) == dt
    a = ops.relayout(qt, torch.from_numpy(raw).cuda(), n, rows, cols)
    b = ops.relayout(dt, torch.from_numpy(conv(raw)).cuda(), n, rows, cols)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("name,M", [("tiny_q4_0", 1), ("tiny_q4_0", 16), ("qwen3_q4_0", 1), ("qwen3_q4_0", 300),
                                    ("tiny_q5_0", 1), ("tiny_q5_0", 40), ("tiny_q4_1", 1), ("tiny_q4_1", 40),
                                    ("qwen3_q4_1", 4), ("qwen3_q4_1", 8), ("qwen3_q4_1", 700)])
def test_q4_0_layer(name, M):
    from pgmoe import HipSparseMoEMLP
    spec = {"tiny_q4_0": LayerSpec("tiny_q4_0", 1024, 8, 2, 512, (Q4_0, Q4_0, Q4_0)),
            "qwen3_q4_0": LayerSpec("qwen3_q4_0", 2048, 128, 8, 768, (Q4_0, Q4_0, Q4_0)),
            "tiny_q5_0": LayerSpec("tiny_q5_0", 1024, 8, 2, 512, (Q5_0, Q5_0, Q4_0)),
            "tiny_q4_1": LayerSpec("tiny_q4_1", 1024, 8, 2, 512, (Q4_1, Q4_1, Q4_1), shared_inter=512,
                                   shared_qtypes=(Q4_1, Q4_1, Q4_1), shared_gate=True, arch="qwen2moe",
                                   norm_topk=False),
            "qwen3_q4_1": LayerSpec("qwen3_q4_1", 2048, 128, 8, 768, (Q4_1, Q4_1, Q6_K))}[name]
    lay = SyntheticLayer(spec, seed=0)
    ol = oracle.OracleLayer.from_gguf(lay.gguf, lay.config)
    mod = HipSparseMoEMLP(lay.gguf, lay.config, 0, torch.device("cuda", 0))
    log(f"q4_0 layer {name} M={M}")
    x = lay.draw_x(M)
    got = mod(torch.from_numpy(x).cuda()).cpu().numpy()
    logits, idx, w = ol.route(x)
    toks = sample_tokens(M, 8)
    stats = check_layer_output(got[toks], ol.forward_tokens(x, idx, w, tokens=toks))
    log(f"  {name} M={M}: {stats}")
