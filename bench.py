"""Benchmark of the quantized-weight matmul path on one MI355X.

Headline (BASELINE.json metric "weight-stream GB/s (% HBM peak) + us per quant matmul at M=1 and
M=8", configs[1]): one step = one rotated MLX-affine 2-bit projection (Ternary Bonsai 27B style,
17408 x 5120, group 64, 128-point Walsh-Hadamard on the input fused into the GEMV) at M=1, over
synthetic seeded weights already resident in HBM. value = algorithmic weight-stream bytes / time
per call (GB/s, 1e9). The weights rotate through >= 600 MB of copies so the 256 MB Infinity Cache
cannot serve them. Calls are captured once into a HIP graph and replayed, so the timed region
holds kernel time, not Python launch overhead.

Also printed (same JSON line, "families"), every BASELINE config at its own shape:
  cfg0  Q4_0 4096x4096, M = 1 and 8
  cfg1  affine 2-bit g64 + WHT 17408x5120, M = 1, 2, 4, 8
  cfg2  Q4_K, Q6_K, IQ2_XS at 25600x5120 (gate/up) and 5120x25600 (down), M = 1 and 8
  cfg3  EXL3 2 bpw 5120 -> 17408, M = 1, 2, 4, 8
  cfg4  MoE FFN, 128 Q4_K experts, H 2048, I 768, top-8, T = 1, 8, 64
and the north-star shape 17408x5120 for Q4_0, Q4_K, Q6_K and IQ2_XS at M = 1 and 8. With --all,
also the other GGUF formats (Q2_K, IQ4_XS, IQ2_XXS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M), the
3- to 8-bit affine packs and the MoE over affine experts. cpu_baseline: the CPU restatement
(oracle/ishz_oracle.c, timed in C: rotate, then dequantize-then-dot; and the fused decode-dot)
on the full headline matrix, OpenMP on the host's cores, median of 10.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12
CACHE_DEFEAT = 600e6


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--all", action="store_true", help="also the other GGUF formats, affine 4/8-bit and MoE over "
                                                       "affine experts")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma list of family names to run (debug)")
    ap.add_argument("--ceiling", action="store_true",
                    help="only the read ceiling: a plain streaming read (ishz_stream_read) of 16 MB .. 600 MB, "
                         "one JSON line")
    ap.add_argument("--policy", action="store_true",
                    help="measure the row-count dispatch policy (VerifyMatmul.minimumRows, ggmlApply's "
                         "row ranges) instead of the benchmark")
    return ap.parse_args()


def policy():
    """Row-count dispatch re-measured on MI355X (one JSON line).

    affine (VerifyMatmul.minimumRows, Core/VerifyMatmul.swift:19-26): per weight size, us for one
    M-row verify call vs M one-row GEMV calls; minimum_rows = fewest rows (2..8) where the verify
    call wins. GGUF Q4_K (ggmlApply, Core/Hadamard.swift:145-178): us for one matvec call with M
    rows (M <= 16), for ceil(M/16) 16-row calls, and for dequantize + fp16 GEMM (hipBLAS through
    torch.matmul); crossover = fewest rows where the dense path wins. Weights are uniform random
    codes made on the device (timing does not depend on their values)."""
    import numpy as np
    import torch

    from ishizuki_amd import _lib
    from ishizuki_amd._torch import ptr

    L = _lib.lib()
    dev = torch.device("cuda:0")
    st = lambda: torch.cuda.current_stream().cuda_stream

    def us(fn, reps=40):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000 / reps

    out = {"metric": "row-count dispatch policy on MI355X", "affine": [], "q4_k": []}
    g = torch.Generator(device=dev).manual_seed(5)
    for name, N, K in (("attn k/v", 1024, 5120), ("6144-wide", 6144, 5120), ("mlp", 17408, 5120),
                       ("output head", 248320, 5120)):
        codes = torch.randint(-2**31, 2**31 - 1, (N, K // 16), dtype=torch.int32, device=dev, generator=g)
        sc = (torch.rand((N, K // 64), device=dev, generator=g) * 0.02).half()
        bi = -sc
        x = torch.randn((8, K), device=dev, generator=g).half()
        y = torch.empty((8, N), device=dev, dtype=torch.half)
        call = lambda M: L.ishz_affine_matmul(ptr(x), 1, M, K, ptr(codes), ptr(sc), ptr(bi), 1, N, 2, 64, ptr(y), st())
        one = us(lambda: call(1))
        row = {"shape": f"{N}x{K}", "what": name, "weight_bytes": codes.numel() * 4 + sc.numel() * 4,
               "gemv_us": round(one, 2), "verify_us": {}}
        mr = None
        for M in range(2, 9):
            if call(M) != 0:  # declined: no time to report
                row["verify_us"][M] = None
                continue
            t = us(lambda: call(M))
            row["verify_us"][M] = round(t, 2)
            if mr is None and t < M * one:
                mr = M
        row["minimum_rows"] = mr
        out["affine"].append(row)
        del codes, sc, bi
    for name, N, K in (("attn k/v", 1024, 5120), ("mlp up", 25600, 5120), ("mlp down", 5120, 25600)):
        nb = N * (K // 256) * 144
        blk = torch.randint(0, 256, (nb,), dtype=torch.uint8, device=dev, generator=g)
        blk.view(-1, 144)[:, :4] = torch.tensor([0x1f, 0x1c, 0x1f, 0x1c], dtype=torch.uint8, device=dev)  # d, dmin ~ 0.005
        x = torch.randn((64, K), device=dev, generator=g).half()
        y = torch.empty((64, N), device=dev, dtype=torch.half)
        wd = torch.empty((N, K), device=dev, dtype=torch.half)
        mv = lambda M, r0=0: L.ishz_ggml_matvec(12, ptr(x[r0:]), 1, M, K, ptr(blk), nb, N, ptr(y[r0:]), st())

        def chunks(M):
            for r0 in range(0, M, 16):
                mv(min(16, M - r0), r0)

        def dense(M):
            L.ishz_ggml_dequant(12, ptr(blk), nb, N * K, ptr(wd), 1, st())
            torch.matmul(x[:M], wd.t(), out=y[:M])

        row = {"shape": f"{N}x{K}", "what": name, "weight_bytes": nb, "matvec_us": {}, "chunks16_us": {},
               "dense_us": {}}
        cross = None
        for M in (1, 2, 4, 8, 12, 16, 24, 32, 48, 64):
            if M <= 16:
                row["matvec_us"][M] = round(us(lambda: mv(M)), 2)
            tc = us(lambda: chunks(M))
            td = us(lambda: dense(M))
            row["chunks16_us"][M] = round(tc, 2)
            row["dense_us"][M] = round(td, 2)
            if cross is None and td < tc:
                cross = M
        row["dense_from_rows"] = cross
        out["q4_k"].append(row)
        del blk, wd
    print(json.dumps(out))


def main():
    args = parse()
    if args.policy:
        return policy()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the kernels shard by "
              "output rows, each GPU its own slice of y). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from ishizuki_amd import affine, exl3, ggml, moe, synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    def copies_of(nbytes):
        return max(2, int(np.ceil(CACHE_DEFEAT / max(nbytes, 1))))

    def timed(calls, steps, warmup):
        """Capture one pass over `calls` (one per weight copy) in a HIP graph, and the first
        steps % len(calls) of them in a second one; time exactly `steps` calls (whole passes, then
        the remainder). Returns seconds per call (events on the capture stream) and the count."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for c in calls:  # first call outside capture (lazy init), checks the result exists
                c()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        steps = max(1, steps)
        full, rem = divmod(steps, len(calls))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for c in calls:
                c()
        g2 = None
        if rem:
            g2 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g2):
                for c in calls[:rem]:
                    c()
        for _ in range(max(1, (warmup + len(calls) - 1) // len(calls))):
            g.replay()
        torch.cuda.synchronize()
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        for _ in range(full):
            g.replay()
        if g2 is not None:
            g2.replay()
        en.record()
        torch.cuda.synchronize()
        return st.elapsed_time(en) * 1e-3 / steps, steps

    # ------------------------------------------------------------------ workloads
    def ggml_case(t, N, K, M, seed=1):
        blk = torch.from_numpy(synth.ggml_blocks(t, N, K, seed=seed)).to(dev)
        nb = blk.numel()
        ws = [blk] + [blk.clone() for _ in range(copies_of(nb) - 1)]
        x = torch.from_numpy(synth.fp16_normal((M, K), seed=seed + 1)).to(dev)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        L = ggml._lib.lib()
        from ishizuki_amd._torch import ptr
        wsb = L.ishz_ggml_workspace_size(t, M, K, N)  # K-split parts for narrow outputs (M >= 2)
        wsp = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        calls = [lambda w=w: L.ishz_ggml_matvec_ws(t, ptr(x), 1, M, K, ptr(w), nb, N, ptr(y), ptr(wsp), wsb,
                                                   torch.cuda.current_stream().cuda_stream) for w in ws]
        return calls, nb, nb + 2 * M * (K + N)

    def affine_case(N, K, M, seed=2):
        codes, s, b = synth.affine_pack(N, K, group=64, seed=seed)
        c0 = torch.from_numpy(codes.view(np.int32)).to(dev)
        s0, b0 = torch.from_numpy(s).to(dev), torch.from_numpy(b).to(dev)
        nb = c0.numel() * 4 + s0.numel() * 2 + b0.numel() * 2
        sets = [(c0, s0, b0)] + [(c0.clone(), s0.clone(), b0.clone()) for _ in range(copies_of(nb) - 1)]
        x = torch.from_numpy(synth.fp16_normal((M, K), seed=seed + 1)).to(dev)
        signs = torch.from_numpy(synth.hadamard_signs(K, seed=seed + 2)).to(dev)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        L = affine._lib.lib()
        from ishizuki_amd._torch import ptr
        wsb = L.ishz_affine_workspace_size(M, K)
        wsp = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        calls = [lambda c=c, sc=sc, bi=bi: L.ishz_affine_linear(
            ptr(x), 1, M, K, ptr(signs), 128, ptr(c), ptr(sc), ptr(bi), 1, N, 2, 64, ptr(y), ptr(wsp), wsb,
            torch.cuda.current_stream().cuda_stream) for c, sc, bi in sets]
        return calls, nb, nb + 2 * M * (K + N)

    def read_case(nbytes):
        """A plain streaming read of the same byte count (ishz_stream_read): the practical ceiling
        for a kernel that reads those bytes once."""
        n16 = (nbytes + 15) // 16 * 16
        bufs = [torch.empty(n16, dtype=torch.uint8, device=dev).fill_(1) for _ in range(copies_of(n16))]
        sink = torch.zeros(1, dtype=torch.int32, device=dev)
        L = affine._lib.lib()
        from ishizuki_amd._torch import ptr
        calls = [lambda b=b: L.ishz_stream_read(ptr(b), n16, ptr(sink), torch.cuda.current_stream().cuda_stream)
                 for b in bufs]
        return calls, n16, n16

    def affine_nbit_case(N, K, M, bits, seed=6):
        """Plain (unrotated) 4- or 8-bit MLX affine pack, g64: ishz_affine_matmul."""
        codes, s, b = synth.affine_pack_bits(N, K, bits, group=64, seed=seed)
        c0 = torch.from_numpy(codes.view(np.int32)).to(dev)
        s0, b0 = torch.from_numpy(s).to(dev), torch.from_numpy(b).to(dev)
        nb = c0.numel() * 4 + s0.numel() * 2 + b0.numel() * 2
        sets = [(c0, s0, b0)] + [(c0.clone(), s0.clone(), b0.clone()) for _ in range(copies_of(nb) - 1)]
        x = torch.from_numpy(synth.fp16_normal((M, K), seed=seed + 1)).to(dev)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        L = affine._lib.lib()
        from ishizuki_amd._torch import ptr
        calls = [lambda c=c, sc=sc, bi=bi: L.ishz_affine_matmul(
            ptr(x), 1, M, K, ptr(c), ptr(sc), ptr(bi), 1, N, bits, 64, ptr(y), torch.cuda.current_stream().cuda_stream)
            for c, sc, bi in sets]
        return calls, nb, nb + 2 * M * (K + N)

    def exl3_case(K, N, M, bits2=4, seed=3):
        t, suh, svh = synth.exl3_pack(K, N, bits2=bits2, seed=seed)
        t0 = torch.from_numpy(t).to(dev)
        su, sv = torch.from_numpy(suh).to(dev), torch.from_numpy(svh).to(dev)
        nb = t0.numel() * 2
        ts = [t0] + [t0.clone() for _ in range(copies_of(nb) - 1)]
        x = torch.from_numpy(synth.fp16_normal((M, K), seed=seed + 1)).to(dev)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        L = exl3._lib.lib()
        from ishizuki_amd._torch import ptr
        wsb = L.ishz_exl3_workspace_size(M, K, N)
        wsp = torch.empty(wsb, dtype=torch.uint8, device=dev)
        calls = [lambda tt=tt: L.ishz_exl3_apply(ptr(x), 1, M, K, ptr(tt), ptr(su), ptr(sv), N, bits2, 0, ptr(y),
                                                 ptr(wsp), wsb, torch.cuda.current_stream().cuda_stream) for tt in ts]
        return calls, nb + 2 * (K + N), nb + 2 * (K + N) + 2 * M * (K + N)

    def moe_case(T, E=128, H=2048, I=768, k=8, seed=4, scale=4e-4):
        # super-scales |N| * 4e-4 rather than the config's |N| * 0.01: with uniformly random 6-bit
        # sub-scales the latter overflows fp16 in the SwiGLU intermediates (outputs inf); timing
        # does not depend on the values, and the outputs are checked finite before timing
        gate = synth.ggml_blocks(ggml.Q4_K, E * I, H, seed=seed, scale=scale)
        up = synth.ggml_blocks(ggml.Q4_K, E * I, H, seed=seed + 1, scale=scale)
        down = synth.ggml_blocks(ggml.Q4_K, E * H, I, seed=seed + 2, scale=scale)
        ex = moe.GGMLExperts(*(torch.from_numpy(a).to(dev) for a in (gate, up, down)), ggml.Q4_K, E, H, I)
        pool = 3 * ex.expert_bytes * E
        exs = [ex] + [moe.GGMLExperts(ex.gate.clone(), ex.up.clone(), ex.down.clone(), ggml.Q4_K, E, H, I)
                      for _ in range(copies_of(pool) - 1)]
        x = torch.from_numpy(synth.fp16_normal((T, H), seed=seed + 3)).to(dev)
        logits_np = np.random.default_rng(seed + 5).standard_normal((T, E)).astype(np.float32)
        logits = torch.from_numpy(logits_np).to(dev)
        # distinct experts this seed routes to (top-k of the logits = top-k of the softmax)
        distinct = len(np.unique(np.argsort(-logits_np, axis=1, kind="stable")[:, :k]))
        y = torch.empty((T, H), dtype=torch.float16, device=dev)
        L = moe._lib.lib()
        from ishizuki_amd._torch import ptr
        wsb = L.ishz_moe_workspace_size(T, H, E, I, k)
        wsp = torch.empty(wsb, dtype=torch.uint8, device=dev)
        calls = [lambda e=e: L.ishz_moe_swiglu(ggml.Q4_K, ptr(x), 1, T, H, ptr(logits), E, k, 1, ptr(e.gate),
                                               ptr(e.up), ptr(e.down), e.expert_bytes, I, None, None, ptr(y), None, None,
                                               ptr(wsp), wsb, torch.cuda.current_stream().cuda_stream) for e in exs]
        calls[0]()
        torch.cuda.synchronize()
        assert bool(torch.isfinite(y).all()), "MoE bench outputs must be finite"
        nb = distinct * 3 * ex.expert_bytes
        return calls, nb, nb, distinct

    def moe_affine_case(T, E=128, H=2048, I=768, k=8, bits=4, seed=8):
        """The MoE FFN over MLX affine stacked experts (4-bit g64), weights made on the device."""
        g = torch.Generator(device=dev).manual_seed(seed)

        def pack(rows, K):
            c = torch.randint(-2**31, 2**31 - 1, (E, rows, K * bits // 32), dtype=torch.int32, device=dev, generator=g)
            sc = (torch.rand((E, rows, K // 64), device=dev, generator=g) * 0.01).half()
            return c, sc, (-sc.float() * (1 << (bits - 1))).half()
        packs = (pack(I, H), pack(I, H), pack(H, I))
        per_expert = sum(p[0].numel() * 4 + p[1].numel() * 2 + p[2].numel() * 2 for p in packs) // E
        copies = [packs] + [tuple(tuple(t.clone() for t in p) for p in packs)
                            for _ in range(copies_of(per_expert * E) - 1)]
        x = torch.from_numpy(synth.fp16_normal((T, H), seed=seed + 3)).to(dev)
        logits_np = np.random.default_rng(seed + 5).standard_normal((T, E)).astype(np.float32)
        logits = torch.from_numpy(logits_np).to(dev)
        distinct = len(np.unique(np.argsort(-logits_np, axis=1, kind="stable")[:, :k]))
        y = torch.empty((T, H), dtype=torch.float16, device=dev)
        L = moe._lib.lib()
        from ishizuki_amd._torch import ptr
        wsb = L.ishz_moe_workspace_size(T, H, E, I, k)
        wsp = torch.empty(wsb, dtype=torch.uint8, device=dev)
        calls = [lambda c=c: L.ishz_moe_swiglu_affine(
            ptr(x), 1, T, H, ptr(logits), E, k, 1, *(ptr(t) for p in c for t in p), 1, bits, 64, I, None, None, ptr(y),
            None, None,
            ptr(wsp), wsb, torch.cuda.current_stream().cuda_stream) for c in copies]
        nb = distinct * per_expert
        return calls, nb, nb, distinct

    def measure(name, builder, M, steps, warmup, extra=None, nk=None):
        out = builder()
        calls, wbytes, allbytes = out[0], out[1], out[2]
        sec, n = timed(calls, steps, warmup)
        r = {"name": name, "M": M, "us": round(sec * 1e6, 3), "weight_bytes": int(wbytes),
             "GBps": round(wbytes / sec / 1e9, 1), "hbm_frac": round(wbytes / sec / HBM_PEAK, 4)}
        if nk and M >= 2:  # verify: useful FLOP = 2 M N K against the 2.5 PFLOP/s dense fp16 MFMA peak
            flops = 2.0 * M * nk[0] * nk[1]
            r.update({"TFLOPs": round(flops / sec / 1e12, 2), "mfma_frac": round(flops / sec / 2.5e15, 4),
                      "bytes_per_flop": round(wbytes / flops, 4)})
        if extra:
            r.update(extra(out))
        del out, calls
        torch.cuda.empty_cache()
        return r, sec, n

    ceilings = {}

    def ceiling(nbytes, steps):
        """(us, GB/s) of a plain streaming read of nbytes (cached per byte count)."""
        if nbytes not in ceilings:
            r, _, _ = measure("stream_read", lambda: read_case(nbytes), 1, steps, args.warmup)
            ceilings[nbytes] = (r["us"], r["GBps"])
        return ceilings[nbytes]

    if args.ceiling:
        rows = []
        for mb in (16, 22.28, 25.76, 27.85, 50.14, 65.5, 73.11, 100, 131.1, 200, 340, 600):
            us_, gbps = ceiling(int(mb * 1e6) // 16 * 16, args.steps)
            rows.append({"MB": mb, "us": us_, "GBps": gbps, "hbm_frac": round(gbps * 1e9 / HBM_PEAK, 4)})
        print(json.dumps({"metric": "read ceiling: ishz_stream_read per byte count (graph replay, >= 600 MB "
                                    "of copies)", "rows": rows}), flush=True)
        return

    only = set(filter(None, args.only.split(",")))
    NS, KS = 17408, 5120
    families = []

    # headline: rotated affine 2-bit, M=1 -- one launch of the GEMV (x rotated in its staging), so
    # the call is the roofline kernel; beside it a plain read of the same bytes
    head, head_sec, head_n = measure("affine2_g64_wht128", lambda: affine_case(NS, KS, 1), 1, args.steps, args.warmup)
    rd, rd_sec, _ = measure("stream_read", lambda: read_case(head["weight_bytes"]), 1, args.steps, args.warmup)
    ceilings[int(head["weight_bytes"]) // 16 * 16] = (rd["us"], rd["GBps"])

    fam_steps = max(50, args.steps // 2)

    def add(tag, name, builder, M, shape, nk=None, extra=None):
        if only and name not in only:
            return
        r, _, _ = measure(name, builder, M, fam_steps, args.warmup, nk=nk, extra=extra)
        r["config"] = tag
        r["shape"] = shape
        # the practical ceiling at this family's byte count: a plain streaming read of as many bytes
        cu, cg = ceiling(int(r["weight_bytes"]) // 16 * 16, fam_steps)
        r["read_ceiling_us"], r["read_ceiling_GBps"] = cu, cg
        r["frac_of_read_ceiling"] = round(cu / r["us"], 4)
        families.append(r)

    # cfg0: GGUF Q4_0 4096x4096
    for M in (1, 8):
        add("cfg0", "q4_0", lambda M=M: ggml_case(ggml.Q4_0, 4096, 4096, M), M, "4096x4096", nk=(4096, 4096))
    # cfg1: the headline family at every drafted row count
    for M in (1, 2, 4, 8):
        add("cfg1", "affine2_g64_wht128", lambda M=M: affine_case(NS, KS, M), M, f"{NS}x{KS}", nk=(NS, KS))
    # cfg2: K- and i-quants at the Qwen-27B MLP shapes
    for t, nm in ((ggml.Q4_K, "q4_k"), (ggml.Q6_K, "q6_k"), (ggml.IQ2_XS, "iq2_xs")):
        for (N, K) in ((25600, 5120), (5120, 25600)):
            for M in (1, 8):
                add("cfg2", nm, lambda t=t, N=N, K=K, M=M: ggml_case(t, N, K, M), M, f"{N}x{K}", nk=(N, K))
    # cfg3: EXL3 2 bpw
    for M in (1, 2, 4, 8):
        add("cfg3", "exl3_2bpw", lambda M=M: exl3_case(KS, NS, M), M, f"{NS}x{KS}", nk=(NS, KS))
    # cfg4: MoE FFN
    for T in (1, 8, 64):
        add("cfg4", "moe_q4k_e128_h2048_i768_top8", lambda T=T: moe_case(T), T, "E128 H2048 I768 k8",
            extra=lambda o: {"distinct_experts": int(o[3])})
    # the north-star shape for the GGUF formats
    for t, nm in ((ggml.Q4_0, "q4_0"), (ggml.Q4_K, "q4_k"), (ggml.Q6_K, "q6_k"), (ggml.IQ2_XS, "iq2_xs")):
        for M in (1, 8):
            add("northstar", nm, lambda t=t, M=M: ggml_case(t, NS, KS, M), M, f"{NS}x{KS}", nk=(NS, KS))
    if args.all:
        for bits in (3, 4, 5, 6, 8):
            for M in (1, 8):
                add("extra", f"affine{bits}_g64", lambda M=M, bits=bits: affine_nbit_case(NS, KS, M, bits), M,
                    f"{NS}x{KS}", nk=(NS, KS))
        for t in (ggml.Q2_K, ggml.IQ4_XS, ggml.IQ2_XXS, ggml.IQ2_S, ggml.IQ3_XXS, ggml.IQ3_S, ggml.IQ1_S, ggml.IQ1_M):
            for M in (1, 8):
                add("extra", ggml.NAMES[t].lower(), lambda t=t, M=M: ggml_case(t, NS, KS, M), M, f"{NS}x{KS}",
                    nk=(NS, KS))
        for T in (1, 8, 64):
            add("extra", "moe_affine4_g64_e128_h2048_i768_top8", lambda T=T: moe_affine_case(T), T,
                "E128 H2048 I768 k8", extra=lambda o: {"distinct_experts": int(o[3])})

    # ------------------------------------------------------------------ CPU baseline
    cpu = None
    if not args.no_cpu:
        import ctypes

        import oracle
        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count() or 1
        codes, sc, bi = synth.affine_pack(NS, KS, group=64, seed=2)
        xh = synth.fp16_normal((1, KS), seed=3).view(np.uint16)
        signs = synth.hadamard_signs(KS, seed=4)
        yc = np.zeros(NS, np.float32)
        P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
        L = oracle.lib()
        med = {}
        for variant in (0, 1):
            med[variant] = L.ishzo_bench_affine_linear(P(xh), KS, P(signs), 128, P(codes.view(np.uint32)),
                                                       P(sc.view(np.uint16)), P(bi.view(np.uint16)), NS, 64,
                                                       variant, 10, threads, P(yc))
        wb = head["weight_bytes"]
        cpu = {"value": round(wb / med[0] / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "us_per_call": round(med[0] * 1e6, 1),
               "sample": f"the full headline call ({NS}x{KS}, M=1): oracle/ishz_oracle.c rotate + dequantize-then-"
                         f"fp32-dot, OpenMP {threads} threads, median of 10 calls timed in C",
               "fused_decode_dot": {"value": round(wb / med[1] / 1e9, 3), "us_per_call": round(med[1] * 1e6, 1)}}

    us = head_sec * 1e6
    line = {
        "metric": "weight-stream GB/s (% HBM peak) + µs per quant matmul at M=1 and M=8",
        "value": head["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head_n,
        "warmup": args.warmup,
        "ms_per_step": round(us / 1000, 6),
        "us_per_call": round(us, 3),
        "hbm_frac": head["hbm_frac"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",  # the dot's operands (x and the decoded weights); sums in fp32, codes 2-bit
        "data": "synthetic (seeded): BASELINE configs[1] distributions",
        "config": {"workload": "MLX affine 2-bit g64 + 128-pt WHT GEMV, 17408x5120, M=1 (BASELINE configs[1])",
                   "N": NS, "K": KS, "M": 1, "group": 64, "hadamard_block": 128,
                   "arith": "fp16 x and decoded weights, fp32 accumulation, 2-bit codes",
                   "weight_bytes": head["weight_bytes"], "cache_defeat_bytes": int(CACHE_DEFEAT)},
        # dominant (and only) kernel of the headline call: gemv_kernel<FAffine<64, false>>, HIP
        # events over graph replays; algorithmic bytes = codes + scales + biases. read_ceiling: a
        # plain streaming read of the same byte count, timed the same way.
        "roofline": {"bound": "hbm", "achieved": head["GBps"], "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": head["hbm_frac"], "traffic": _traffic(), "kernel": "gemv_kernel<FAffine<64, false>>",
                     "kernel_us": round(us, 3), "read_ceiling": rd["GBps"], "read_ceiling_us": rd["us"],
                     "frac_of_read_ceiling": round(rd_sec / head_sec, 4)},
        "cpu_baseline": cpu,
        "families": families,
    }
    print(json.dumps(line), flush=True)


def _traffic():
    """HBM bytes per launch of the headline kernel, from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by a copy kernel of known size), or None if absent."""
    p = os.path.join(ROOT, "profiles", "traffic_affine2_gemv_17408x5120.json")
    if not os.path.exists(p):
        return None
    try:
        return json.load(open(p)).get("bytes_per_launch")
    except Exception:
        return None


if __name__ == "__main__":
    main()
