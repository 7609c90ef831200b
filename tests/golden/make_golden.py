"""Write tests/golden/ref_vectors.npz from the reference's own CPU code path.

Run once, in the development container only (the reference tree is not present on the
GPU box and is never shipped):

    python tests/golden/make_golden.py /root/reference

What is recorded (inputs and the reference's outputs, nothing else):

* block decode: Q4_K / Q6_K / Q8_0 random blocks -> the reference's repacked W4 / W8
  arrays (quant_kernels.py:854-982) and its dense weights, read back through its own
  CPU matmul with an fp32 identity input (quant_kernels.py:1276-1291, :1408-1420);
* quantized matmul: fp16 x times those weights through exec_w4a16/w8a16_matmul (CPU);
* activation: exec_fused_act_mul_rowscale on large fp16 gate/up so the row-scale fires
  (quant_kernels.py:1423-1475);
* MoE block: GGUFSparseMoEMLP(gguf_file, config, 0, cpu).forward(x) (model.py:849-937)
  on three tiny layers written with pgmoe's GGUF writer and read by the reference's
  GGUFFile: qwen3moe (Q4_K gate/up, Q6_K down), qwen2moe (Q8_0 + sigmoid-gated shared
  expert, no top-k renorm) and mixtral (all Q4_K), at realistic weight scale so the
  reference's fp16 intermediates stay finite; M = 1 and 16.
"""

from __future__ import annotations

import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "pytorch-engine_amd"))

from pgmoe.gguf import GGUFWriter, GGMLType  # noqa: E402
from pgmoe.synth import LayerSpec, SyntheticLayer, random_blocks  # noqa: E402

Q4_K, Q6_K, Q8_0 = GGMLType.Q4_K, GGMLType.Q6_K, GGMLType.Q8_0

LAYERS = {
    "qwen3moe": LayerSpec("g_qwen3moe", 256, 4, 2, 256, (Q4_K, Q4_K, Q6_K)),
    "qwen2moe": LayerSpec("g_qwen2moe", 256, 4, 2, 128, (Q8_0, Q8_0, Q8_0), norm_topk=False,
                          arch="qwen2moe", shared_inter=256, shared_gate=True),
    "mixtral": LayerSpec("g_mixtral", 256, 4, 2, 256, (Q4_K, Q4_K, Q4_K), arch="mixtral"),
}


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import torch
    from pygguf_engine import quant_kernels as qk
    from pygguf_engine.gguf_parser import GGUFFile as RefGGUFFile
    from pygguf_engine.model import GGUFSparseMoEMLP

    cpu = torch.device("cpu")
    out: dict = {}
    rng = np.random.default_rng(20240601)

    # ---- block decode + quantized matmul -------------------------------------------
    rows, cols = 4, 512
    x = (rng.standard_normal((5, cols), dtype=np.float32) * 0.5).astype(np.float16)
    out["mm_x"] = x
    for name, qt in (("q4_k", Q4_K), ("q6_k", Q6_K), ("q8_0", Q8_0)):
        for tag, scale in (("big", 1.0), ("small", 0.01)):
            raw = random_blocks(rng, qt, rows, cols, scale)
            key = f"{name}_{tag}"
            out[f"dq_{key}_raw"] = raw
            eye = torch.eye(cols, dtype=torch.float32)
            if qt == Q4_K:
                qw, sc, zr = qk.repack_gguf_to_w4a16(raw, int(qt), rows, cols, cpu)
                dense = qk.exec_w4a16_matmul(eye, qw, sc, zr).T.contiguous()
                out[f"dq_{key}_zeros"] = zr.numpy()
                mm = qk.exec_w4a16_matmul(torch.from_numpy(x), qw, sc, zr)
            else:
                qw, sc, zr = qk.repack_gguf_to_w8a16(raw, int(qt), rows, cols, cpu)
                assert zr is None
                dense = qk.exec_w8a16_matmul(eye, qw, sc, None).T.contiguous()
                mm = qk.exec_w8a16_matmul(torch.from_numpy(x), qw, sc, None)
            out[f"dq_{key}_qweight"] = qw.numpy()
            out[f"dq_{key}_scales"] = sc.numpy()
            out[f"dq_{key}_dense"] = dense.numpy()
            if tag == "small":
                out[f"mm_{name}_out"] = mm.numpy()

    # ---- activation + row-scale ---------------------------------------------------
    g = (rng.standard_normal((3, 300), dtype=np.float32) * 200.0).astype(np.float16)
    u = (rng.standard_normal((3, 300), dtype=np.float32) * 200.0).astype(np.float16)
    din, rsc = qk.exec_fused_act_mul_rowscale(torch.from_numpy(g), torch.from_numpy(u))
    out["act_g"], out["act_u"] = g, u
    out["act_down_in"], out["act_row_scale"] = din.numpy(), rsc.numpy()

    # ---- MoE block forward ----------------------------------------------------------
    with tempfile.TemporaryDirectory() as td:
        for lname, spec in LAYERS.items():
            layer = SyntheticLayer(spec, seed=7, scale=0.01)
            path = os.path.join(td, f"{lname}.gguf")
            w = GGUFWriter()
            for k, v in layer.gguf.metadata.items():
                w.add_meta(k, v)
            w.add_meta(f"{spec.arch}.block_count", 1)
            for tname, info in layer.gguf.tensors.items():
                w.add_tensor(tname, info.shape, info.qtype, layer.gguf.get_tensor_bytes(tname))
                out[f"moe_{lname}__{tname}"] = np.array(layer.gguf.get_tensor_bytes(tname))
            w.write(path)
            gf = RefGGUFFile(path)
            cfg = gf.build_model_config()
            assert cfg.n_experts == spec.n_experts and cfg.n_experts_used == spec.top_k
            assert cfg.norm_topk_prob == spec.norm_topk
            mod = GGUFSparseMoEMLP(gf, cfg, 0, cpu)
            for M in (1, 16):
                xm = layer.draw_x(M)
                xt = torch.from_numpy(xm).view(1, M, spec.hidden)
                with torch.inference_mode():
                    y = mod(xt)
                    probs = torch.softmax(torch.nn.functional.linear(xt.view(M, -1).float(),
                                                                     mod.router_weight), dim=-1)
                    tw, ti = torch.topk(probs, k=mod.top_k, dim=-1)
                out[f"moe_{lname}_M{M}_x"] = xm
                out[f"moe_{lname}_M{M}_out"] = y.reshape(M, spec.hidden).float().numpy()
                out[f"moe_{lname}_M{M}_topk_idx"] = ti.numpy().astype(np.int32)
                out[f"moe_{lname}_M{M}_logits"] = torch.nn.functional.linear(
                    xt.view(M, -1).float(), mod.router_weight).numpy()
            out[f"moe_{lname}_meta"] = np.array([spec.hidden, spec.n_experts, spec.top_k, spec.inter,
                                                 int(spec.norm_topk), spec.shared_inter], dtype=np.int64)
            del mod
            gf.close()

    dst = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({os.path.getsize(dst)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
