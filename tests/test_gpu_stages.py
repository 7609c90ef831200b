"""GPU parity of the individual C-ABI stages against the CPU oracle.

Integer/index stages (router logits in their fixed order, top-k ids, dispatch) must be
bit-exact; floating-point stages are checked with the tolerances stated per test.
"""

import numpy as np
import pytest

import oracle
from gpu_helpers import log
from pgmoe.synth import random_blocks

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q4_1, Q4_K, Q5_K, Q6_K, Q8_0 = 3, 12, 13, 14, 8


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)


def _np_relayout(qtype, raw, n_mats, rows, cols, stride):
    """The device layout of include/pgmoe.h (64-row tiles of 16-byte chunks), in numpy."""
    out = np.zeros(n_mats * stride, dtype=np.uint8)
    nb, ng = cols // 256, (rows + 63) // 64
    bpb = {Q4_1: 160, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_0: 272}[qtype]  # GGUF bytes per 256 weights
    CH = {Q4_1: 10, Q4_K: 9, Q5_K: 11, Q6_K: 13, Q8_0: 17}[qtype]
    sb = raw.reshape(n_mats, rows, nb, bpb)
    for m in range(n_mats):
        base = m * stride
        for r in range(rows):
            g, rr = divmod(r, 64)
            for b in range(nb):
                blk = sb[m, r, b]
                t = base + (g * nb + b) * CH * 1024 + rr * 16
                if qtype == Q4_1:  # d's, m's, then the codes in the Q4_K arrangement
                    for j in range(8):
                        bj = blk[20 * j:20 * j + 20]
                        out[t + 2 * j:t + 2 * j + 2] = bj[0:2]
                        out[t + 1024 + 2 * j:t + 1024 + 2 * j + 2] = bj[2:4]
                    code = np.concatenate([np.concatenate([blk[20 * j + 4:20 * j + 20] & 15, blk[20 * j + 4:20 * j + 20] >> 4])
                                           for j in range(8)])  # element 32j + l
                    qs = np.array([code[64 * (k >> 5) + (k & 31)] | (code[64 * (k >> 5) + 32 + (k & 31)] << 4)
                                   for k in range(128)], dtype=np.uint8)
                    for c in range(8):
                        out[t + (2 + c) * 1024:t + (2 + c) * 1024 + 16] = qs[16 * c:16 * c + 16]
                elif qtype == Q5_K:  # header + qs as Q4_K, then the fifth bits per quarter
                    for c in range(9):
                        src = 0 if c == 0 else 48 + 16 * (c - 1)
                        out[t + c * 1024:t + c * 1024 + 16] = blk[src:src + 16]
                    qh = blk[16:48].astype(np.uint64)
                    for p in range(4):
                        for tt in range(2):
                            word = 0
                            for l in range(32):
                                word |= int((qh[l] >> np.uint64(2 * p + tt)) & np.uint64(1)) << (8 * (l & 3) + (l >> 2))
                            o = t + (9 + (p >> 1)) * 1024 + 8 * (p & 1) + 4 * tt
                            out[o:o + 4] = np.array([word], dtype="<u4").view(np.uint8)
                elif qtype in (Q4_K, Q6_K):
                    for c in range(CH):
                        out[t + c * 1024:t + c * 1024 + 16] = blk[16 * c:16 * c + 16]
                    if qtype == Q6_K:
                        d = base + ng * nb * CH * 1024 + ((g * nb + b) * 64 + rr) * 2
                        out[d:d + 2] = blk[208:210]
                else:
                    for j in range(8):
                        bj = blk[34 * j:34 * j + 34]
                        out[t + 2 * j * 1024:t + 2 * j * 1024 + 16] = bj[2:18]
                        out[t + (2 * j + 1) * 1024:t + (2 * j + 1) * 1024 + 16] = bj[18:34]
                        out[t + 16 * 1024 + 2 * j:t + 16 * 1024 + 2 * j + 2] = bj[0:2]
    return out


@pytest.mark.parametrize("qtype,rows,cols,n_mats", [(Q4_K, 8, 512, 3), (Q6_K, 7, 768, 3), (Q8_0, 5, 256, 2),
                                                    (Q6_K, 130, 768, 2), (Q8_0, 64, 512, 1), (Q5_K, 70, 512, 2),
                                                    (Q4_1, 70, 512, 2)])
def test_relayout_bytes(dev, qtype, rows, cols, n_mats):
    from pgmoe import ops
    rng = np.random.default_rng(rows * cols)
    raw = np.concatenate([random_blocks(rng, qtype, rows, cols) for _ in range(n_mats)])
    buf = ops.relayout(qtype, torch.from_numpy(raw).to(dev), n_mats, rows, cols)
    stride = ops.weight_stride(qtype, rows, cols)
    got = buf.cpu().numpy()
    ref = _np_relayout(qtype, raw, n_mats, rows, cols, stride)
    # bytes past the tiles (alignment padding between matrices) are unspecified
    ng, nb = (rows + 63) // 64, cols // 256
    mb = ng * nb * {Q4_1: 10 * 1024, Q4_K: 9 * 1024, Q5_K: 11 * 1024, Q6_K: 13 * 1024 + 128, Q8_0: 17 * 1024}[qtype]
    for m in range(n_mats):
        assert np.array_equal(got[m * stride:m * stride + mb], ref[m * stride:m * stride + mb])


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, Q8_0])
def test_relayout_unaligned_source(dev, qtype):
    """A source view that does not start 16-byte aligned (the kernels read 16-byte aligned
    rows): ops.relayout copies it first, and the bytes match the aligned source's."""
    from pgmoe import ops
    rows, cols = 70, 512
    raw = random_blocks(np.random.default_rng(7), qtype, rows, cols)
    base = torch.zeros(raw.size + 2, dtype=torch.uint8, device=dev)
    base[2:] = torch.from_numpy(raw).to(dev)
    view = base[2:]
    assert view.data_ptr() % 16 != 0
    got = ops.relayout(qtype, view, 1, rows, cols).cpu().numpy()
    ref = ops.relayout(qtype, torch.from_numpy(raw).to(dev), 1, rows, cols).cpu().numpy()
    ng, nb = (rows + 63) // 64, cols // 256  # the tiles (padding past them is unspecified)
    mb = ng * nb * {Q4_K: 9 * 1024, Q6_K: 13 * 1024 + 128, Q8_0: 17 * 1024}[qtype]
    assert np.array_equal(got[:mb], ref[:mb])


@pytest.mark.parametrize("M,H,E,K,bias", [(1, 2048, 128, 8, False), (8, 2048, 128, 8, False),
                                          (333, 2048, 128, 8, True), (4096, 2048, 128, 8, True),
                                          (5, 1024, 8, 2, False), (64, 3584, 64, 8, False),
                                          (17, 4096, 8, 2, False), (3, 512, 512, 16, False),
                                          (40, 1024, 24, 4, True),
                                          # the small-grid tiles: 4 x 2 (Mixtral's E = 8) and 1 x 1
                                          (2048, 4096, 8, 2, False), (512, 3584, 1, 1, False),
                                          (300, 1024, 3, 2, True),
                                          # grouped top-k at its bounds (32 lanes a token: E = 128,
                                          # K = 16; 16 lanes: E = 32; M not a multiple of a block's
                                          # tokens), a whole wave a token past them (K = 20; E = 129)
                                          (37, 512, 128, 16, True), (21, 512, 32, 16, True),
                                          (33, 512, 100, 20, False), (19, 512, 129, 8, True)])
def test_router_topk_bitexact(dev, M, H, E, K, bias):
    from pgmoe import ops
    log(f"router M={M} H={H} E={E} K={K}")
    rng = np.random.default_rng(M + H + E)
    x = rng.standard_normal((M, H), dtype=np.float32).astype(np.float16)
    w = (rng.standard_normal((E, H), dtype=np.float32) * 0.02).astype(np.float32)
    b = rng.standard_normal(E).astype(np.float32) if bias else None
    lg, idx, tw = ops.router_topk(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev),
                                  None if b is None else torch.from_numpy(b).to(dev), K, True)
    ref_lg = oracle.router_logits(x, w, b)
    ref_idx, ref_w = oracle.topk(ref_lg, K, True)
    assert np.array_equal(lg.cpu().numpy().view(np.uint32), ref_lg.view(np.uint32))
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    np.testing.assert_allclose(tw.cpu().numpy(), ref_w, rtol=2e-6, atol=1e-7)
    _, _, tw2 = ops.router_topk(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev),
                                None if b is None else torch.from_numpy(b).to(dev), K, False)
    _, ref_w2 = oracle.topk(ref_lg, K, False)
    np.testing.assert_allclose(tw2.cpu().numpy(), ref_w2, rtol=2e-6, atol=1e-8)


def test_topk_ties_lower_id_wins(dev):
    from pgmoe import ops
    H, E, K, M = 512, 16, 4, 6
    x = np.zeros((M, H), np.float16)
    x[:, 0] = 1.0
    w = np.zeros((E, H), np.float32)
    w[:, 0] = np.array([1, 3, 3, 2, 3, 0, 3, 1, 2, 2, 0, 0, 3, 1, 1, 2], np.float32)
    _, idx, _ = ops.router_topk(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev), None, K, True)
    assert np.all(idx.cpu().numpy() == np.array([1, 2, 4, 6], np.int32))


@pytest.mark.parametrize("blocks", ["one", "many"])
@pytest.mark.parametrize("M,K,E,skew", [(1, 8, 128, None), (8, 8, 128, None), (4096, 8, 128, None),
                                        (4096, 8, 128, "one"), (16, 2, 8, None), (1000, 1, 1, None),
                                        (512, 8, 64, "half"), (3, 16, 512, None), (0, 8, 128, None),
                                        (20000, 8, 128, None), (300, 7, 9, "one")])
def test_dispatch_bitexact(dev, M, K, E, skew, blocks):
    """pgmoe_dispatch (one workgroup) and pgmoe_dispatch_ws (a counting pass, then up to 64
    scatter workgroups; M = 20000 exceeds that cap) against a stable argsort."""
    from pgmoe import ops
    log(f"dispatch M={M} K={K} E={E} skew={skew} blocks={blocks}")
    rng = np.random.default_rng(M * 7 + K)
    idx = np.array([rng.permutation(E)[:K] for _ in range(M)], dtype=np.int32).reshape(M, K)
    if skew == "one" and M:
        idx[:, 0] = 5  # every token picks expert 5 ...
        for t in range(M):  # ... keeping ids distinct per token
            row = [e for e in rng.permutation(E) if e != 5][:K - 1]
            idx[t, 1:] = row
    if skew == "half" and M:
        idx = np.stack([np.sort(rng.permutation(E // 2)[:K]) for _ in range(M)]).astype(np.int32)
    offsets, perm, inv, active, n_active, tile_off = ops.dispatch(torch.from_numpy(idx).to(dev), E, 64, blocks)
    r_off, r_perm, r_inv = oracle.dispatch(idx, E)
    assert np.array_equal(offsets.cpu().numpy(), r_off)
    assert np.array_equal(perm.cpu().numpy(), r_perm)
    assert np.array_equal(inv.cpu().numpy(), r_inv)
    counts = np.diff(r_off)
    act = np.nonzero(counts)[0]
    assert int(n_active.cpu()[0]) == len(act)
    assert np.array_equal(active.cpu().numpy()[:len(act)], act)
    tiles = (counts + 63) // 64
    assert np.array_equal(tile_off.cpu().numpy(), np.concatenate([[0], np.cumsum(tiles)]))


def _dense(qtype, raw, n_mats, rows, cols):
    return oracle.dequant(qtype, raw, n_mats * rows, cols).reshape(n_mats, rows, cols).astype(np.float64)


def _np_scale_plane(qtype, raw, n_mats, rows, cols):
    """The scale plane of include/pgmoe.h in numpy (fp32, the kernel's expressions and
    operation order): per (64-row group, super-block, unit c) 64 rows of four floats."""
    nb, ng = cols // 256, (rows + 63) // 64
    bpb = {Q4_1: 160, Q4_K: 144, Q5_K: 176, Q6_K: 210}[qtype]
    sb = np.zeros((n_mats, ng * 64, nb, bpb), dtype=np.uint8)  # pad rows: zero bytes
    sb[:, :rows] = raw.reshape(n_mats, rows, nb, bpb)
    out = np.zeros((n_mats, ng, nb, 4, 64, 4), dtype=np.float32)
    f32 = np.float32
    for m in range(n_mats):
        for r in range(ng * 64):
            g, rr = divmod(r, 64)
            for b in range(nb):
                blk = sb[m, r, b]
                for c in range(4):
                    if qtype == Q4_1:  # a = d, c = m - 1024 a of blocks 2c, 2c + 1
                        vals = []
                        for s in (2 * c, 2 * c + 1):
                            dq, mq = blk[20 * s:20 * s + 4].view(np.float16).astype(np.float32)
                            vals += [f32(dq), f32(mq) - f32(1024.0) * f32(dq)]
                    elif qtype in (Q4_K, Q5_K):
                        d, dmin = blk[0:4].view(np.float16).astype(np.float32)
                        q = blk[4:16].astype(np.int64)
                        vals = []
                        for s in (2 * c, 2 * c + 1):
                            if s < 4:
                                sc, mn = q[s] & 63, q[s + 4] & 63
                            else:
                                sc = (q[s + 4] & 0xF) | ((q[s - 4] >> 6) << 4)
                                mn = (q[s + 4] >> 4) | ((q[s] >> 6) << 4)
                            a = f32(d) * f32(sc)
                            vals += [a, -(f32(dmin) * f32(mn)) - f32(1024.0) * a]
                    else:
                        d = blk[208:210].view(np.float16).astype(np.float32)[0]
                        scl = blk[192:208].view(np.int8)
                        h, half = c >> 1, c & 1
                        vals = [f32(d) * f32(scl[8 * h + 2 * gg + half]) for gg in range(4)]
                    out[m, g, b, c, rr] = vals
    return out.reshape(n_mats, -1)


@pytest.mark.parametrize("qtype,rows,cols,n_mats", [(Q4_K, 8, 512, 3), (Q6_K, 7, 768, 3), (Q4_K, 130, 256, 2),
                                                    (Q5_K, 70, 512, 2), (Q4_1, 70, 512, 2)])
def test_scale_plane_bits(dev, qtype, rows, cols, n_mats):
    """The load-time scale plane equals its numpy restatement bit for bit (pad rows too)."""
    from pgmoe import ops
    rng = np.random.default_rng(rows + cols)
    raw = np.concatenate([random_blocks(rng, qtype, rows, cols) for _ in range(n_mats)])
    buf = ops.relayout(qtype, torch.from_numpy(raw).to(dev), n_mats, rows, cols)
    plane = ops.scale_plane(qtype, buf, n_mats, rows, cols)
    torch.cuda.synchronize()
    got = plane.cpu().numpy().view(np.uint32).reshape(n_mats, -1)
    ref = _np_scale_plane(qtype, raw, n_mats, rows, cols).view(np.uint32)
    bad = np.argwhere(got != ref)
    assert len(bad) == 0, (len(bad), bad[:4].tolist(), got[tuple(bad[0])], ref[tuple(bad[0])])
    assert ops.scale_plane(Q8_0, buf, 1, 64, 256) is None  # Q8_0 has no plane


def test_mfma_products_need_the_scale_plane(dev):
    """Mode 1 (MFMA) with K-quant weights but no scale plane is an error, not a fallback."""
    from pgmoe import ops
    rng = np.random.default_rng(3)
    E, I, H, K, M = 2, 64, 256, 1, 16
    gb = ops.relayout(Q4_K, torch.from_numpy(np.concatenate([random_blocks(rng, Q4_K, I, H) for _ in range(E)])).to(dev),
                      E, I, H)
    W = ops.make_weights(Q4_K, gb, E, I, H)
    idx = torch.zeros((M, K), dtype=torch.int32, device=dev)
    disp = ops.dispatch(idx, E, 256)
    x = torch.zeros((M, H), dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="scale plane"):
        ops.expert_gateup(W, W, x, K, disp, 1)


@pytest.mark.parametrize("qg,qd,H,I,E,K,M,mode", [
    (Q4_K, Q6_K, 512, 256, 8, 2, 1, 0), (Q4_K, Q6_K, 512, 256, 8, 2, 8, 0),
    (Q4_K, Q4_K, 256, 512, 4, 2, 5, 0), (Q8_0, Q8_0, 256, 512, 6, 3, 7, 0),
    (Q6_K, Q8_0, 768, 256, 3, 1, 6, 0), (Q4_K, Q6_K, 2304, 512, 5, 2, 8, 0),
    (Q4_K, Q6_K, 512, 256, 8, 2, 40, 1), (Q4_K, Q4_K, 256, 512, 4, 2, 130, 1),
    (Q8_0, Q8_0, 256, 512, 6, 3, 70, 1), (Q6_K, Q8_0, 256, 256, 3, 1, 9, 1),
    (Q4_K, Q6_K, 512, 256, 8, 2, 3, 1), (Q8_0, Q4_K, 512, 256, 3, 2, 17, 1),
    (Q5_K, Q5_K, 512, 256, 8, 2, 1, 0), (Q5_K, Q5_K, 256, 512, 4, 2, 8, 0), (Q5_K, Q6_K, 768, 512, 5, 2, 6, 0),
    (Q5_K, Q5_K, 512, 256, 8, 2, 40, 1), (Q5_K, Q5_K, 256, 512, 4, 2, 130, 1), (Q6_K, Q5_K, 512, 256, 3, 1, 9, 1),
    (Q4_1, Q4_1, 512, 256, 8, 2, 1, 0), (Q4_1, Q4_1, 256, 512, 4, 2, 8, 0), (Q4_1, Q6_K, 512, 256, 8, 2, 40, 1),
    (Q4_1, Q4_1, 256, 512, 4, 2, 130, 1)])
def test_expert_stages(dev, qg, qd, H, I, E, K, M, mode):
    """inter and the weighted down partials against float64 numpy over decoded weights.
    Tolerance: the decode GEMV forms exact fp16 products of (1024 + code) and x and
    removes the 1024 * sum(x) offset after fp32 accumulation, which costs ~2e-5 rel-L2
    (bound 1e-4); the MFMA GEMM uses fp16 weights/x and a per-row fp16 down input
    (rel-L2 2e-3, i.e. fp16 rounding, as in the reference's own GPU prefill path)."""
    from pgmoe import ops
    log(f"stages qg={qg} qd={qd} H={H} I={I} E={E} K={K} M={M} mode={mode}")
    rng = np.random.default_rng(H + I + M)
    gr = np.concatenate([random_blocks(rng, qg, I, H) for _ in range(E)])
    ur = np.concatenate([random_blocks(rng, qg, I, H) for _ in range(E)])
    dr = np.concatenate([random_blocks(rng, qd, H, I) for _ in range(E)])
    x = rng.standard_normal((M, H), dtype=np.float32).astype(np.float16)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(M)]).astype(np.int32)
    tw = rng.random((M, K)).astype(np.float32)
    gb = ops.relayout(qg, torch.from_numpy(gr).to(dev), E, I, H)
    ub = ops.relayout(qg, torch.from_numpy(ur).to(dev), E, I, H)
    db = ops.relayout(qd, torch.from_numpy(dr).to(dev), E, H, I)
    gp, up_, dp = (ops.scale_plane(qg, gb, E, I, H), ops.scale_plane(qg, ub, E, I, H),
                   ops.scale_plane(qd, db, E, H, I))
    Wg, Wu = ops.make_weights(qg, gb, E, I, H, gp), ops.make_weights(qg, ub, E, I, H, up_)
    Wd = ops.make_weights(qd, db, E, H, I, dp)
    disp = ops.dispatch(torch.from_numpy(idx).to(dev), E, 256)  # the GEMM's tile size
    xd = torch.from_numpy(x).to(dev)
    inter = ops.expert_gateup(Wg, Wu, xd, K, disp, mode)
    tw_d = torch.from_numpy(tw).to(dev)
    partial = ops.expert_down(Wd, inter, M, K, disp, tw_d, mode)
    torch.cuda.synchronize()
    _, perm, _ = oracle.dispatch(idx, E)
    g = _dense(qg, gr, E, I, H)
    u = _dense(qg, ur, E, I, H)
    d = _dense(qd, dr, E, H, I)
    xf = x.astype(np.float64)
    P = M * K
    ref_inter = np.empty((P, I))
    for p in range(P):
        f = perm[p]
        t, k = divmod(int(f), K)
        e = idx[t, k]
        gv, uv = g[e] @ xf[t], u[e] @ xf[t]
        ref_inter[p] = gv / (1 + np.exp(-gv)) * uv
    got_inter = inter.cpu().numpy()
    tol = 1e-4 if mode == 0 else 2e-3
    assert oracle.rel_l2(got_inter, ref_inter) < tol, ("inter", oracle.rel_l2(got_inter, ref_inter))
    ref_part = np.empty((P, H))
    gi = got_inter.astype(np.float64)
    for p in range(P):
        t, k = divmod(int(perm[p]), K)
        ref_part[p] = tw[t, k] * (d[idx[t, k]] @ gi[p])
    assert oracle.rel_l2(partial.cpu().numpy(), ref_part) < tol
    assert oracle.max_rel(partial.cpu().numpy(), ref_part) < 50 * tol


@pytest.mark.parametrize("I", [1024, 4096, 14336, 20480])
def test_rowscale_bit_exact_and_down(dev, I):
    """The prefill down stage's row-scale (exec_fused_act_mul_rowscale's second half,
    quant_kernels.py:1467-1475): rs = max(max|v| / 16384, 1) and a16 = fp16(v / rs) bit for bit
    against numpy, for the one-wave rows (I <= 4096) and the one-block rows (Mixtral's 14336,
    Qwen2's shared 20480), with rows large enough to scale; then the down partials within the
    MFMA tolerance."""
    from pgmoe import ops
    log(f"rowscale I={I}")
    rng = np.random.default_rng(I)
    H, E, K, M = 256, 4, 2, 40
    P = M * K
    dr = np.concatenate([random_blocks(rng, Q8_0, H, I, 0.1) for _ in range(E)])
    db = ops.relayout(Q8_0, torch.from_numpy(dr).to(dev), E, H, I)
    Wd = ops.make_weights(Q8_0, db, E, H, I, ops.scale_plane(Q8_0, db, E, H, I))
    idx = np.stack([rng.permutation(E)[:K] for _ in range(M)]).astype(np.int32)
    tw = rng.random((M, K)).astype(np.float32)
    disp = ops.dispatch(torch.from_numpy(idx).to(dev), E, 256)
    inter = rng.standard_normal((P, I)).astype(np.float32)
    inter[::3] *= np.float32(3e4)  # every third row above the fp16-safe range: rs > 1
    inter[1, 7] = np.float32(-7e6)  # a row whose maximum is a single negative value
    a16 = torch.empty((P, I), dtype=torch.float16, device=dev)
    rs = torch.empty(P, dtype=torch.float32, device=dev)
    partial = ops.expert_down(Wd, torch.from_numpy(inter).to(dev), M, K, disp, torch.from_numpy(tw).to(dev), 1,
                              rowscale=(a16, rs))
    torch.cuda.synchronize()
    ref_rs = np.maximum(np.abs(inter).max(axis=1) * np.float32(1.0 / 16384.0), np.float32(1.0)).astype(np.float32)
    ref_a16 = (inter / ref_rs[:, None]).astype(np.float16)
    assert np.array_equal(rs.cpu().numpy().view(np.uint32), ref_rs.view(np.uint32))
    assert np.array_equal(a16.cpu().numpy().view(np.uint16), ref_a16.view(np.uint16))
    assert (ref_rs > 1).sum() >= P // 3
    _, perm, _ = oracle.dispatch(idx, E)
    d = _dense(Q8_0, dr, E, H, I)
    ref_part = np.empty((P, H))
    a64 = ref_a16.astype(np.float64) * ref_rs[:, None].astype(np.float64)
    for p in range(P):
        t, k = divmod(int(perm[p]), K)
        ref_part[p] = tw[t, k] * (d[idx[t, k]] @ a64[p])
    assert oracle.rel_l2(partial.cpu().numpy(), ref_part) < 2e-3


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 8, 16])  # the sorting networks (K <= 4) and the selection
def test_combine_order_and_shared(dev, K):
    from pgmoe import ops
    rng = np.random.default_rng(5 + K)
    M, H, E = 9, 128, 16
    idx = np.stack([rng.permutation(E)[:K] for _ in range(M)]).astype(np.int32)
    _, perm, inv = oracle.dispatch(idx, E)
    part = rng.standard_normal((M * K, H)).astype(np.float32) * np.float32(1e4)
    sh = rng.standard_normal((M, H)).astype(np.float32)
    slog = rng.standard_normal(M).astype(np.float32)
    out = ops.combine(torch.from_numpy(part).to(dev), torch.from_numpy(inv).to(dev), M, K,
                      torch.from_numpy(sh).to(dev), torch.from_numpy(slog).to(dev)).cpu().numpy()
    ref = np.zeros((M, H), np.float32)
    for t in range(M):
        acc = np.zeros(H, np.float32)
        for k in np.argsort(idx[t], kind="stable"):  # ascending expert id
            acc = acc + part[inv[t * K + k]]
        gate = np.float32(1.0) / (np.float32(1.0) + np.exp(-slog[t]))
        ref[t] = acc + sh[t] * gate
    np.testing.assert_allclose(out, ref, rtol=1e-6, atol=1e-6)
    # routed part alone is summed in ascending expert order: bitwise
    out2 = ops.combine(torch.from_numpy(part).to(dev), torch.from_numpy(inv).to(dev), M, K).cpu().numpy()
    ref2 = np.zeros((M, H), np.float32)
    for t in range(M):
        acc = np.zeros(H, np.float32)
        for k in np.argsort(idx[t], kind="stable"):
            acc = acc + part[inv[t * K + k]]
        ref2[t] = acc
    assert np.array_equal(out2, ref2)
