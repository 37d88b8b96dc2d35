"""Teacher-forced forward parity (test infrastructure).

`StepForward` replays the engine's forward (the launch sequence of eva_forward in xtagger_amd/csrc/engine.cpp, itself
src/engine/eva.h:227-310) kernel by kernel through the C-ABI on torch buffers, with the weights packed on the GPU
exactly as the engine's bring-up does. After every kernel it hands the step's GPU inputs and outputs to `check`,
which recomputes the step with the oracle *from the GPU's own inputs* and compares. Each step is therefore pinned
at its real shape, and the engine's graph is then shown to produce the same bits as this validated sequence.

Why teacher forcing: every block re-quantizes its activations to E4M3 (6% steps). Two implementations whose fp32
sums differ only in order (the oracle's scalar and AVX2 loops, or the matrix core) flip a few roundings, and the
flipped values change the next layer's sums, so free-running forwards of the same model drift apart to the level of
the quantization noise within a few layers. The oracle shows this against itself; see test_forward_gpu.py.
"""
import numpy as np
import torch

T, D, TP, HIDP, HID = 1025, 1024, 1088, 2816, 2730


class StepForward:
    """sparse: the four layer GEMMs' packed weights are 2:4-pruned and packed (eva_k_prune24 / eva_k_pack24) and the
    sparse kernels run, as the engine does with EVA_SPARSE24."""

    def __init__(self, xt, m, nb, dev, sparse=False):
        self.xt, self.m, self.nb, self.dev, self.sparse = xt, m, nb, dev, sparse
        self.M = nb * T
        self.lds = (self.M + 255) // 256 * 256
        self.st = torch.cuda.current_stream().cuda_stream
        L, P, st = xt.lib, xt.ptr, self.st
        up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        self.pe, self.pos, self.cs = up(m["pe"]), up(m["pos"]), up(m["rope"])
        self.fnw, self.fnb = up(m["fnw"]), up(m["fnb"])
        scratch = torch.empty(2 * HIDP * D, dtype=torch.float32, device=dev)
        self.layers = []
        for Lw in m["layers"]:
            d = {k: up(Lw[k]) for k in ("ln1w", "ln1b", "ln2w", "ln2b", "mlnw", "mlnb")}
            w16 = {k: up(Lw[k]) for k in ("wqkv", "wo", "w12", "w2")}
            z8 = lambda *s: torch.zeros(*s, dtype=torch.uint8, device=dev)
            zf = lambda *s: torch.zeros(*s, dtype=torch.float32, device=dev)
            d["wqkv"], d["sqkv"] = z8(3 * D, D), zf(24, 8)
            d["wo"], d["so"] = z8(D, D), zf(8, 8)
            d["w12"], d["s12"] = z8(2 * HIDP, D), zf(44, 8)
            d["w2"], d["s2"] = z8(D, HIDP), zf(8, 22)
            d["cn"], d["dn"] = zf(D), zf(D)
            ck = lambda rc: xt.check(rc, "prep")
            ck(L.eva_k_prep_w(P(w16["wqkv"]), D, 3 * D, D, 3 * D, D, 1, None, P(scratch), P(d["wqkv"]), P(d["sqkv"]), st))
            ck(L.eva_k_prep_w(P(w16["wo"]), D, D, D, D, D, 0, None, P(scratch), P(d["wo"]), P(d["so"]), st))
            ck(L.eva_k_prep_w(P(w16["w12"]), D, 2 * 2736, D, 2 * HIDP, D, 0, None, P(scratch), P(d["w12"]), P(d["s12"]),
                              st))
            ck(L.eva_k_prep_w(P(w16["w2"]), 2736, D, HID, D, HIDP, 0, P(d["mlnw"]), P(scratch), P(d["w2"]), P(d["s2"]),
                              st))
            if sparse:
                for k, n, kk in (("wqkv", 3 * D, D), ("wo", D, D), ("w12", 2 * HIDP, D), ("w2", D, HIDP)):
                    ck(L.eva_k_prune24(P(d[k]), n, kk, st))
                    d[k + "_v"] = z8(n // 16, kk // 128, 64, 16)
                    d[k + "_x"] = torch.zeros(n // 16, kk // 128, 64, dtype=torch.int32, device=dev)
                    ck(L.eva_k_pack24(P(d[k]), n, kk, P(d[k + "_v"]), P(d[k + "_x"]), None, st))
            ck(L.eva_k_fold_cd(P(d["w2"]), P(d["s2"]), P(w16["w2"]), 2736, P(d["mlnb"]), P(d["cn"]), P(d["dn"]), st))
            torch.cuda.synchronize()
            self.layers.append(d)
        nt = m["nt"]
        self.nt = nt
        hw16 = up(m["hw"][:nt])
        self.ldh = (nt + 63) // 64 * 64
        self.hq = torch.zeros(nt, D, dtype=torch.uint8, device=dev)
        self.hs = torch.zeros(8, self.ldh, dtype=torch.float32, device=dev)
        self.hb = up(m["hb"][:nt])
        # the head rows each packed with their own 1x128 scales, as the engine's bring-up does
        xt.check(L.eva_k_quant_act(P(hw16), 2, D, nt, D, P(self.hq), D, P(self.hs), self.ldh, st), "head")
        torch.cuda.synchronize()
        M, lds = self.M, self.lds
        self.x = torch.zeros(lds, D, dtype=torch.int16, device=dev)
        self.h8 = torch.zeros(lds, D, dtype=torch.uint8, device=dev)
        self.sh = torch.zeros(8, lds, dtype=torch.float32, device=dev)
        self.q = torch.zeros(nb, 16, TP, 64, dtype=torch.int16, device=dev)
        self.k = torch.zeros_like(self.q)
        self.vt = torch.zeros(nb, 16, 64, TP, dtype=torch.int16, device=dev)
        self.o32 = torch.zeros(M, D, dtype=torch.float32, device=dev)
        self.m8 = torch.zeros(lds, HIDP, dtype=torch.uint8, device=dev)
        self.sm = torch.zeros(22, lds, dtype=torch.float32, device=dev)
        self.stat = torch.zeros(22, lds, 2, dtype=torch.float32, device=dev)
        self.pool = torch.zeros(nb, D, dtype=torch.float32, device=dev)
        self.pn = torch.zeros(nb, D, dtype=torch.int16, device=dev)
        self.pq = torch.zeros(nb, D, dtype=torch.uint8, device=dev)
        self.ps = torch.zeros(8, nb, dtype=torch.float32, device=dev)
        self.out = torch.zeros(nb, nt, dtype=torch.float32, device=dev)

    def run(self, inp, check=None, nl=24):
        """Forward of fp16 inputs [nb][1024][592]; check(step, layer, gpu) after each kernel (gpu: dict of host
        copies of that step's inputs and outputs)."""
        xt, L, P, st, M, lds, nb = self.xt, self.xt.lib, self.xt.ptr, self.st, self.M, self.lds, self.nb
        h = lambda t: t.cpu().numpy()
        sync = torch.cuda.synchronize
        d_in = torch.from_numpy(np.ascontiguousarray(inp)).to(self.dev)
        xt.check(L.eva_k_pe(P(d_in), P(self.pe), P(self.pos), P(self.x), nb, st), "pe")
        sync()
        if check:
            check("pe", -1, {"x": h(self.x[:M])})
        for i, W in enumerate(self.layers[:nl]):
            x0 = h(self.x[:M]) if check else None
            xt.check(L.eva_k_ln(P(self.x), P(W["ln1w"]), P(W["ln1b"]), P(self.h8), P(self.sh), M, lds, st), "ln1")
            sync()
            if check:
                check("ln1", i, {"x": x0, "h8": h(self.h8[:M]), "sh": h(self.sh[:, :M])})
                a8, as_ = h(self.h8[:M]), h(self.sh[:, :M])
            if self.sparse:
                xt.check(L.eva_k_qkv_sp(P(self.h8), P(self.sh), lds, P(W["wqkv_v"]), P(W["wqkv_x"]), P(W["sqkv"]),
                                        P(self.cs), P(self.q), P(self.k), P(self.vt), M, st), "qkv")
            else:
                xt.check(L.eva_k_qkv(P(self.h8), P(self.sh), lds, P(W["wqkv"]), P(W["sqkv"]), P(self.cs), P(self.q),
                                     P(self.k), P(self.vt), M, st), "qkv")
            sync()
            if check:
                check("qkv", i, {"h8": a8, "sh": as_, "q": h(self.q), "k": h(self.k), "vt": h(self.vt)})
            xt.check(L.eva_k_flash(P(self.q), P(self.k), P(self.vt), P(self.h8), P(self.sh), lds, nb, P(self.o32), st),
                     "flash")
            sync()
            if check:
                check("flash", i, {"q": h(self.q), "k": h(self.k), "vt": h(self.vt), "o32": h(self.o32),
                                   "h8": h(self.h8[:M]), "sh": h(self.sh[:, :M])})
                a8, as_, x1 = h(self.h8[:M]), h(self.sh[:, :M]), h(self.x[:M])
            if self.sparse:
                xt.check(L.eva_k_oproj_sp(P(self.h8), P(self.sh), lds, P(W["wo_v"]), P(W["wo_x"]), P(W["so"]),
                                          P(self.x), M, st), "oproj")
            else:
                xt.check(L.eva_k_oproj(P(self.h8), P(self.sh), lds, P(W["wo"]), P(W["so"]), P(self.x), M, st), "oproj")
            sync()
            if check:
                check("oproj", i, {"h8": a8, "sh": as_, "x_in": x1, "x": h(self.x[:M])})
                x2 = h(self.x[:M])
            xt.check(L.eva_k_ln(P(self.x), P(W["ln2w"]), P(W["ln2b"]), P(self.h8), P(self.sh), M, lds, st), "ln2")
            sync()
            if check:
                check("ln2", i, {"x": x2, "h8": h(self.h8[:M]), "sh": h(self.sh[:, :M])})
                a8, as_ = h(self.h8[:M]), h(self.sh[:, :M])
            if self.sparse:
                xt.check(L.eva_k_fc1_sp(P(self.h8), P(self.sh), lds, P(W["w12_v"]), P(W["w12_x"]), P(W["s12"]),
                                        P(self.m8), P(self.sm), P(self.stat), M, st), "fc1")
            else:
                xt.check(L.eva_k_fc1(P(self.h8), P(self.sh), lds, P(W["w12"]), P(W["s12"]), P(self.m8), P(self.sm),
                                     P(self.stat), M, st), "fc1")
            sync()
            if check:
                check("fc1", i, {"h8": a8, "sh": as_, "m8": h(self.m8[:M]), "sm": h(self.sm[:, :M]),
                                 "stat": h(self.stat[:, :M])})
                m8, ms, stt, x3 = h(self.m8[:M]), h(self.sm[:, :M]), h(self.stat[:, :M]), h(self.x[:M])
            if self.sparse:
                xt.check(L.eva_k_fc2_sp(P(self.m8), P(self.sm), lds, P(W["w2_v"]), P(W["w2_x"]), P(W["s2"]),
                                        P(self.stat), P(W["cn"]), P(W["dn"]), P(self.x), M, st), "fc2")
            else:
                xt.check(L.eva_k_fc2(P(self.m8), P(self.sm), lds, P(W["w2"]), P(W["s2"]), P(self.stat), P(W["cn"]),
                                     P(W["dn"]), P(self.x), M, st), "fc2")
            sync()
            if check:
                check("fc2", i, {"m8": m8, "sm": ms, "stat": stt, "x_in": x3, "x": h(self.x[:M])})
        xt.check(L.eva_k_pool(P(self.x), P(self.pool), nb, st), "pool")
        xt.check(L.eva_k_lnh(P(self.pool), P(self.fnw), P(self.fnb), P(self.pn), P(self.pq), P(self.ps), nb, nb, st),
                 "lnh")
        xt.check(L.eva_k_head(P(self.pq), P(self.ps), nb, P(self.hq), P(self.hs), self.ldh, P(self.hb), P(self.out),
                              nb, self.nt, st), "head")
        sync()
        if check:
            check("head", nl, {"x": h(self.x[:M]), "pool": h(self.pool), "pn": h(self.pn), "pq": h(self.pq),
                               "ps": h(self.ps), "out": h(self.out)})
        return h(self.out)
