"""MoE expert-gathered quantized FFN on the GPU vs the oracle's loop-per-token restatement
(the reference's own strategy, MoEBlockTests.swift:94-145), through the C ABI.

Routing ids: exact. Routing weights: 1e-6 relative. Output: max|y - ref| <= 1e-3 * max|ref|.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import MOE_ELEM, assert_close, moe_reference
from ishizuki_amd import ggml, moe, synth

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def experts(E, H, I, type_=ggml.Q4_K, seed=0, scale=4e-4):
    # Super-scales well below the benchmark's |N|*0.01 keep the fp16 SwiGLU intermediates finite
    # (with random 6-bit sub-scales that scale overflows fp16 in the down projection).
    gate = synth.ggml_blocks(type_, E * I, H, seed=seed, scale=scale)
    up = synth.ggml_blocks(type_, E * I, H, seed=seed + 1, scale=scale)
    down = synth.ggml_blocks(type_, E * H, I, seed=seed + 2, scale=scale)
    dev = lambda a: torch.from_numpy(a).to(DEV)
    return (gate, up, down), moe.GGMLExperts(dev(gate), dev(up), dev(down), type_, E, H, I)


@pytest.mark.parametrize("T", [1, 3, 64])
def test_route_matches_oracle(T):
    logits = np.random.default_rng(T).standard_normal((T, 128)).astype(np.float32)
    ids, w = moe.route(torch.from_numpy(logits).to(DEV), 8)
    rid, rw = oracle.moe_route(logits, 8)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.allclose(w.cpu().numpy(), rw, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("T,E", [(5, 100), (20, 1000), (3, 64)])
def test_route_ties_and_odd_expert_counts(T, E):
    """Quantised logits (many exact ties: the lower index wins), E not a multiple of 64, and with
    E = 1000 the two-kernel route + place path (the fused one needs 17 key rows in LDS)."""
    r = np.random.default_rng(E + T)
    logits = (np.round(r.standard_normal((T, E)) * 2) / 2).astype(np.float32)
    ids, w = moe.route(torch.from_numpy(logits).to(DEV), 8)
    rid, rw = oracle.moe_route(logits, 8)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.allclose(w.cpu().numpy(), rw, rtol=1e-6, atol=1e-7)
    x = synth.fp16_normal((T, 256), seed=E)
    (g, u, d), ex = experts(E, 256, 256, seed=E)
    y, ids2, w2 = moe.swiglu(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=8,
                             return_routing=True)
    assert np.array_equal(ids2.cpu().numpy(), rid)
    assert np.allclose(w2.cpu().numpy(), rw, rtol=1e-6, atol=1e-7)
    ref, bd = moe_reference(ggml.Q4_K, x.astype(np.float32), rid, rw, g, u, d, E, 256)
    assert_close(y.float().cpu().numpy(), ref, bound=bd, elem=MOE_ELEM, what=f"moe ties T={T} E={E}")


@pytest.mark.parametrize("T,type_", [(1, ggml.Q4_K), (2, ggml.Q4_K), (2, ggml.Q6_K), (1, ggml.Q4_0), (5, ggml.Q4_K), (20, ggml.Q4_K), (4, ggml.Q6_K), (3, ggml.Q4_0)])
def test_swiglu_small(T, type_):
    E, H, I, k = 16, 512, 256, 4
    (g, u, d), ex = experts(E, H, I, type_, seed=T)
    x = synth.fp16_normal((T, H), seed=T + 7)
    logits = np.random.default_rng(T + 9).standard_normal((T, E)).astype(np.float32)
    y, ids, w = moe.swiglu(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k,
                           return_routing=True)
    rid, rw = oracle.moe_route(logits, k)
    assert np.array_equal(ids.cpu().numpy(), rid)
    ref, bd = moe_reference(type_, x.astype(np.float32), rid, rw, g, u, d, E, I)
    assert_close(y.float().cpu().numpy(), ref, bound=bd, elem=MOE_ELEM, what=f"moe T={T}")


@pytest.mark.parametrize("T,E,k", [(3, 4, 2), (16, 4, 2), (16, 64, 16)])
def test_swiglu_routing_inside_gate_up(T, E, k):
    """Three to sixteen tokens: every gate/up workgroup routes and places the pairs itself and
    workgroup (0, 0) publishes them. Few experts (about T k / E pairs each) and a wide I (several
    workgroups per expert, which must agree on the pair order), and the largest pair count this
    path takes (T k = 256); the published ids and weights are checked too."""
    H, I = 512, 1024
    (g, u, d), ex = experts(E, H, I, ggml.Q4_K, seed=90 + T + k)
    x = synth.fp16_normal((T, H), seed=91 + T)
    logits = np.random.default_rng(92 + T + k).standard_normal((T, E)).astype(np.float32)
    y, ids, w = moe.swiglu(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k,
                           return_routing=True)
    rid, rw = oracle.moe_route(logits, k)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.allclose(w.cpu().numpy(), rw, rtol=1e-6, atol=1e-7)
    ref, bd = moe_reference(ggml.Q4_K, x.astype(np.float32), rid, rw, g, u, d, E, I)
    assert_close(y.float().cpu().numpy(), ref, bound=bd, elem=MOE_ELEM, what=f"moe routed in gate/up T={T} E={E} k={k}")


def test_swiglu_many_tokens_per_expert():
    """4 experts, top-2 of 40 tokens: about 20 tokens per expert, more than one 16-token pass."""
    E, H, I, k, T = 4, 512, 256, 2, 40
    (g, u, d), ex = experts(E, H, I, ggml.Q4_K, seed=77)
    x = synth.fp16_normal((T, H), seed=78)
    logits = np.random.default_rng(79).standard_normal((T, E)).astype(np.float32)
    y = moe.swiglu(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k)
    rid, rw = oracle.moe_route(logits, k)
    assert np.bincount(rid.reshape(-1), minlength=E).max() > 16
    ref, bd = moe_reference(ggml.Q4_K, x.astype(np.float32), rid, rw, g, u, d, E, I)
    assert_close(y.float().cpu().numpy(), ref, bound=bd, elem=MOE_ELEM, what="moe many tokens per expert")


@pytest.mark.parametrize("T", [1, 2, 8, 64])
def test_swiglu_qwen_shape(T):
    # Qwen MoE: 128 experts, hidden 2048, expert intermediate 768, top-8;
    # T = 1, 2 take the gathered GEMVs, T = 8 and 64 the streaming MFMA kernels
    print(f"moe qwen T={T}", flush=True)
    E, H, I, k = 128, 2048, 768, 8
    (g, u, d), ex = experts(E, H, I, seed=50)
    x = synth.fp16_normal((T, H), seed=51)
    logits = np.random.default_rng(52).standard_normal((T, E)).astype(np.float32)
    y = moe.swiglu(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k)
    rid, rw = oracle.moe_route(logits, k)
    ref, bd = moe_reference(ggml.Q4_K, x.astype(np.float32), rid, rw, g, u, d, E, I)
    assert_close(y.float().cpu().numpy(), ref, bound=bd, elem=MOE_ELEM, what=f"moe qwen shape T={T}")


def _random_moe_cases(n, seed):
    """Seeded problems: T from 1 to 12 tokens (the gathered GEMVs and the streaming kernels),
    E from 4 to 64 experts, top-k from 1 to min(8, E), H and I multiples of 256 up to 1536, the
    three expert formats in turn."""
    r = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        E = int(r.integers(4, 65))
        cases.append((int(r.integers(1, 13)), E, int(r.integers(1, min(8, E) + 1)), 256 * int(r.integers(1, 7)),
                      256 * int(r.integers(1, 7)), (ggml.Q4_0, ggml.Q4_K, ggml.Q6_K)[i % 3]))
    return cases


@pytest.mark.parametrize("T,E,k,H,I,type_", _random_moe_cases(12, 2027))
def test_swiglu_random_shapes(T, E, k, H, I, type_):
    print(f"moe random T={T} E={E} k={k} H={H} I={I} type={type_}", flush=True)
    (g, u, d), ex = experts(E, H, I, type_, seed=T + E)
    x = synth.fp16_normal((T, H), seed=H + T)
    logits = np.random.default_rng(E + k).standard_normal((T, E)).astype(np.float32)
    y = moe.swiglu(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k)
    assert y is not None
    rid, rw = oracle.moe_route(logits, k)
    ref, bd = moe_reference(type_, x.astype(np.float32), rid, rw, g, u, d, E, I)
    assert_close(y.float().cpu().numpy(), ref, bound=bd, elem=MOE_ELEM,
                 what=f"moe random T={T} E={E} k={k} H={H} I={I} type={type_}")


@pytest.mark.parametrize("T,k", [(2, 32), (1, 64)])
def test_swiglu_large_topk_few_tokens(T, k):
    """Many slots for one or two tokens: past the gathered GEMVs' LDS the per-block kernels run."""
    E, H, I = 64, 512, 768
    (g, u, d), ex = experts(E, H, I, seed=k)
    x = synth.fp16_normal((T, H), seed=k + 1)
    logits = np.random.default_rng(k + 2).standard_normal((T, E)).astype(np.float32)
    y = moe.swiglu(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k)
    assert y is not None
    rid, rw = oracle.moe_route(logits, k)
    ref, bd = moe_reference(ggml.Q4_K, x.astype(np.float32), rid, rw, g, u, d, E, I)
    assert_close(y.float().cpu().numpy(), ref, bound=bd, elem=MOE_ELEM, what=f"moe T={T} k={k}")


def test_declines():
    _, ex = experts(4, 256, 256, seed=1)
    x = torch.zeros((2, 256), dtype=torch.float32, device=DEV)
    assert moe.swiglu(x, torch.zeros((2, 4), device=DEV), ex, top_k=2) is None   # fp32 x


def affine_experts(E, H, I, bits, group, seed, scale):
    def pack(rows, K, s):
        c, sc, b = synth.affine_pack_bits(E * rows, K, bits, group=group, seed=s, scale=scale)
        return c, sc, b
    packs = [pack(I, H, seed), pack(I, H, seed + 1), pack(H, I, seed + 2)]
    dev = lambda a: torch.from_numpy(a).to(DEV)
    tens = [(dev(c.view(np.int32)), dev(sc), dev(b)) for c, sc, b in packs]
    return packs, moe.AffineExperts(tens[0], tens[1], tens[2], bits, group, E, H, I)


def affine_moe_reference(x, rid, rw, packs, E, H, I, bits, group, shared=None, shared_gate=None):
    """The oracle's MoE formula (ishzo_moe_swiglu: fp16 projection outputs, fp16 SwiGLU ops, fp32
    weighted sum in slot order, narrowed once) over affine weights from the oracle's dequantizer."""
    r16 = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32)
    (gc, gs, gb), (uc, us, ub), (dc, ds, db) = packs
    deq = lambda c, s, b, rows, K: oracle.affine_dequant(c, s.view(np.uint16), b.view(np.uint16), E * rows, K, bits,
                                                         group).reshape(E, rows, K)
    Wg, Wu, Wd = deq(gc, gs, gb, I, H), deq(uc, us, ub, I, H), deq(dc, ds, db, H, I)
    T, k = rid.shape
    y = np.zeros((T, H), np.float32)
    for t in range(T):
        acc = np.zeros(H, np.float32)
        for s in range(k):
            e = rid[t, s]
            g = r16(Wg[e] @ x[t]); u = r16(Wu[e] @ x[t])
            sg = r16(1.0 / (1.0 + np.exp(-g)))
            h = r16(r16(g * sg) * u)
            o = r16(Wd[e] @ h)
            acc = (acc + o * np.float32(rw[t, s])).astype(np.float32)
        if shared is not None:
            acc = (acc + r16(r16(1.0 / (1.0 + np.exp(-np.float32(shared_gate[t])))) * shared[t])).astype(np.float32)
        y[t] = r16(acc)
    return y


@pytest.mark.parametrize("T,type_", [(1, ggml.Q4_K), (2, ggml.Q6_K), (8, ggml.Q4_K), (3, ggml.Q4_0)])
def test_swiglu_shared_expert(T, type_):
    """The shared expert's sigmoid(gate) * output, added in fp32 before the one narrowing
    (Text/MoEBlock.swift:158-160): in the two-launch gathered path (T <= 2, combined in the down
    projection's store) and in the streaming path's combine kernel."""
    E, H, I, k = 16, 512, 256, 4
    (g, u, d), ex = experts(E, H, I, type_, seed=T + 40)
    x = synth.fp16_normal((T, H), seed=T + 41)
    logits = np.random.default_rng(T + 42).standard_normal((T, E)).astype(np.float32)
    sh = (synth.fp16_normal((T, H), seed=T + 43).astype(np.float32) * 0.05).astype(np.float16)
    sg = synth.fp16_normal((T,), seed=T + 44)
    y = moe.swiglu(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k,
                   shared=torch.from_numpy(sh).to(DEV), shared_gate=torch.from_numpy(sg).to(DEV))
    rid, rw = oracle.moe_route(logits, k)
    ref, bd = moe_reference(type_, x.astype(np.float32), rid, rw, g, u, d, E, I, shared=sh.astype(np.float32),
                            shared_gate=sg.astype(np.float32))
    assert_close(y.float().cpu().numpy(), ref, bound=bd, elem=MOE_ELEM, what=f"moe shared T={T}")
    with pytest.raises(ValueError):
        moe.swiglu(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k,
                   shared=torch.from_numpy(sh).to(DEV))


@pytest.mark.parametrize("bits,group,T", [(4, 64, 1), (8, 128, 2), (4, 128, 5), (8, 64, 3), (4, 64, 20),
                                          (2, 64, 1), (3, 128, 2), (5, 64, 4), (6, 128, 1), (7, 64, 9), (2, 128, 20),
                                          (3, 64, 1), (6, 64, 6)])
def test_swiglu_affine_experts(bits, group, T):
    """StackedExperts as MLX affine packs (the reference's expert format, any width its
    gatherQuantizedMM takes, Text/MoEBlock.swift:27,48): 2 to 8 bits, weights of about 0.05."""
    E, H, I, k = 16, 512, 256, 4
    packs, ex = affine_experts(E, H, I, bits, group, seed=bits * 10 + T, scale=0.087 / 2 ** (bits - 1))
    x = synth.fp16_normal((T, H), seed=T + 70)
    logits = np.random.default_rng(T + 71).standard_normal((T, E)).astype(np.float32)
    y, ids, w = moe.swiglu_affine(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k,
                                  return_routing=True)
    assert y is not None
    rid, rw = oracle.moe_route(logits, k)
    assert np.array_equal(ids.cpu().numpy(), rid)
    ref = affine_moe_reference(x.astype(np.float32), rid, rw, packs, E, H, I, bits, group)
    assert np.isfinite(ref).all()
    assert_close(y.float().cpu().numpy(), ref, what=f"moe affine bits={bits} g={group} T={T}")


@pytest.mark.parametrize("T", [1, 5])
def test_swiglu_affine_shared_expert(T):
    E, H, I, k, bits, group = 16, 512, 256, 4, 4, 64
    packs, ex = affine_experts(E, H, I, bits, group, seed=90 + T, scale=0.01)
    x = synth.fp16_normal((T, H), seed=T + 91)
    logits = np.random.default_rng(T + 92).standard_normal((T, E)).astype(np.float32)
    sh = (synth.fp16_normal((T, H), seed=T + 93).astype(np.float32) * 0.05).astype(np.float16)
    sg = synth.fp16_normal((T,), seed=T + 94)
    y = moe.swiglu_affine(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k,
                          shared=torch.from_numpy(sh).to(DEV), shared_gate=torch.from_numpy(sg).to(DEV))
    rid, rw = oracle.moe_route(logits, k)
    ref = affine_moe_reference(x.astype(np.float32), rid, rw, packs, E, H, I, bits, group,
                               shared=sh.astype(np.float32), shared_gate=sg.astype(np.float32))
    assert_close(y.float().cpu().numpy(), ref, what=f"moe affine shared T={T}")


def bf16r(a):
    """Values rounded to bf16 (round to nearest even), as float32."""
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def moe_reference_bf16(x, rid, rw, Wg, Wu, Wd, shared=None, shared_gate=None):
    """MoEBlock.callAsFunction + ResidentExperts.swiglu in bf16 (Text/MoEBlock.swift:124-171):
    every projection output and SwiGLU op rounded to bf16, the k slots weighted and summed in
    fp32 in slot order, the shared expert's bf16 term added in fp32, narrowed once. Returns
    (ref, bound) with bound_t = sum_s w_s |Wd[e_s]| @ |h_s| (+ |shared|)."""
    T, k = rid.shape
    H = x.shape[1]
    ref = np.zeros((T, H), np.float32)
    bound = np.zeros((T, H), np.float64)
    for t in range(T):
        acc = np.zeros(H, np.float32)
        for s in range(k):
            e = rid[t, s]
            g = bf16r(Wg[e] @ x[t].astype(np.float64))
            u = bf16r(Wu[e] @ x[t].astype(np.float64))
            with np.errstate(over="ignore"):  # exp(-g) = inf for very negative g: sigmoid 0
                sg = bf16r(1.0 / (1.0 + np.exp(-g.astype(np.float64))))
            h = bf16r(bf16r(g * sg) * u)
            o = bf16r(Wd[e] @ h.astype(np.float64))
            acc = (acc + o * np.float32(rw[t, s])).astype(np.float32)
            bound[t] += float(rw[t, s]) * (np.abs(Wd[e]) @ np.abs(h.astype(np.float64)))
        if shared is not None:
            sgt = bf16r(1.0 / (1.0 + np.exp(-np.float64(shared_gate[t]))))
            acc = (acc + bf16r(sgt * shared[t])).astype(np.float32)
            bound[t] += np.abs(shared[t])
        ref[t] = bf16r(acc)
    return ref, bound


def check_bf16(y, ref, bound, what):
    """bf16 intermediates formed in another summation order may round one bf16 ulp (2^-8) the
    other way: 2^-7 of the bound leaves room for a few such flips; plus the output's own rounding."""
    y = y.float().cpu().numpy().astype(np.float64)
    lim = 2.0 ** -7 * bound + 2.0 ** -8 * np.abs(ref) + 1e-30
    assert np.all(np.isfinite(y)), f"{what}: non-finite"
    bad = np.abs(y - ref) > lim
    assert not bad.any(), f"{what}: {int(bad.sum())} outside; worst {np.max(np.abs(y - ref) / lim):.3g}x"


@pytest.mark.parametrize("T,type_", [(1, ggml.Q4_K), (2, ggml.Q6_K), (5, ggml.Q4_K), (20, ggml.Q4_0), (3, ggml.Q6_K)])
def test_swiglu_bf16(T, type_):
    """The MoE FFN in bf16 (MoEBlock runs in the model's dtype): every stage's bf16 roundings,
    bf16 x and h staged from fp16 images with a factor per row, against a bf16 restatement."""
    E, H, I, k = 16, 512, 256, 4
    (g, u, d), ex = experts(E, H, I, type_, seed=T + 100, scale=0.002)
    x = torch.from_numpy(synth.fp16_normal((T, H), seed=T + 101).astype(np.float32) * 30.0).to(torch.bfloat16)
    logits = np.random.default_rng(T + 102).standard_normal((T, E)).astype(np.float32)
    print(f"moe bf16 T={T} type={type_}", flush=True)
    y, ids, w = moe.swiglu(x.to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k, return_routing=True)
    assert y is not None and y.dtype == torch.bfloat16
    rid, rw = oracle.moe_route(logits, k)
    assert np.array_equal(ids.cpu().numpy(), rid)
    Wg = oracle.dequant_rows(type_, g, E * I, H).reshape(E, I, H).astype(np.float64)
    Wu = oracle.dequant_rows(type_, u, E * I, H).reshape(E, I, H).astype(np.float64)
    Wd = oracle.dequant_rows(type_, d, E * H, I).reshape(E, H, I).astype(np.float64)
    ref, bd = moe_reference_bf16(x.float().numpy(), rid, rw, Wg, Wu, Wd)
    check_bf16(y, ref, bd, f"moe bf16 T={T}")


@pytest.mark.parametrize("T,bits", [(1, 4), (2, 8), (6, 4), (17, 3)])
def test_swiglu_affine_bf16(T, bits):
    """Affine experts (bf16 scales, as a bf16 MLX model ships them) with bf16 activations and the
    shared expert, against the bf16 restatement."""
    E, H, I, k, group = 16, 512, 256, 4, 64
    packs = []
    for i, (rows, K) in enumerate(((I, H), (I, H), (H, I))):
        c, sc, b = synth.affine_pack_bits(E * rows, K, bits, group=group, seed=T + 110 + i, scale=0.087 / 2 ** (bits - 1))
        packs.append((c, bf16r(sc.astype(np.float32)), bf16r(b.astype(np.float32))))
    dev = lambda a: torch.from_numpy(a).to(DEV)
    tens = [(dev(c.view(np.int32)), dev(sc).to(torch.bfloat16), dev(b).to(torch.bfloat16)) for c, sc, b in packs]
    ex = moe.AffineExperts(tens[0], tens[1], tens[2], bits, group, E, H, I)
    x = torch.from_numpy(synth.fp16_normal((T, H), seed=T + 111)).to(torch.bfloat16)
    logits = np.random.default_rng(T + 112).standard_normal((T, E)).astype(np.float32)
    sh = torch.from_numpy(synth.fp16_normal((T, H), seed=T + 113).astype(np.float32) * 0.05).to(torch.bfloat16)
    sg = torch.from_numpy(synth.fp16_normal((T,), seed=T + 114)).to(torch.bfloat16)
    print(f"moe affine bf16 T={T} bits={bits}", flush=True)
    y = moe.swiglu_affine(x.to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k, shared=sh.to(DEV),
                          shared_gate=sg.to(DEV))
    assert y is not None and y.dtype == torch.bfloat16
    rid, rw = oracle.moe_route(logits, k)
    bf16bits = lambda a: torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    W = []
    for (c, sc, b), (rows, K) in zip(packs, ((I, H), (I, H), (H, I))):
        # bf16 scales: the oracle's dequantizer takes fp16 bits, so dequantize in numpy
        q = np.zeros((E * rows, K), np.float64)
        words = c.view(np.uint32).reshape(E * rows, -1).astype(np.uint64)
        for kk in range(K):
            bit = kk * bits
            wv = words[:, bit // 32]
            if bit // 32 + 1 < words.shape[1]:
                wv = wv | (words[:, bit // 32 + 1] << np.uint64(32))
            q[:, kk] = ((wv >> np.uint64(bit % 32)) & np.uint64((1 << bits) - 1)).astype(np.float64)
        s_ = np.repeat(sc.astype(np.float64), group, axis=1)
        b_ = np.repeat(b.astype(np.float64), group, axis=1)
        W.append((s_ * q + b_).astype(np.float32).astype(np.float64).reshape(E, rows, K))
    ref, bd = moe_reference_bf16(x.float().numpy(), rid, rw, *W, shared=sh.float().numpy(),
                                 shared_gate=sg.float().numpy())
    check_bf16(y, ref, bd, f"moe affine bf16 T={T} bits={bits}")


@pytest.mark.parametrize("T", [1, 8, 64])
def test_config4_qwen_moe_bf16(T):
    """BASELINE configs[4] (128 Q4_K experts, H 2048, I 768, top-8) with bf16 activations at
    T = 1, 8 and 64: the gathered GEMVs, the routing-in-gate/up MFMA path, and the routed one
    (routing launch first)."""
    E, H, I, k = 128, 2048, 768, 8
    (g, u, d), ex = experts(E, H, I, ggml.Q4_K, seed=0xB0, scale=4e-4)
    x = torch.from_numpy(synth.fp16_normal((T, H), seed=0xB1 + T)).to(torch.bfloat16)
    logits = np.random.default_rng(0xB2 + T).standard_normal((T, E)).astype(np.float32)
    print(f"config4 bf16 T={T}", flush=True)
    y = moe.swiglu(x.to(DEV), torch.from_numpy(logits).to(DEV), ex, top_k=k)
    assert y is not None and y.dtype == torch.bfloat16
    rid, rw = oracle.moe_route(logits, k)
    bs, ts = 256, 144
    gb, db = I * (H // bs) * ts, H * (I // bs) * ts
    Wg, Wu, Wd = {}, {}, {}  # the routed experts only, float32
    for e in sorted(set(int(e) for e in rid.ravel())):
        Wg[e] = oracle.dequant_rows(ggml.Q4_K, g[e * gb:(e + 1) * gb], I, H)
        Wu[e] = oracle.dequant_rows(ggml.Q4_K, u[e * gb:(e + 1) * gb], I, H)
        Wd[e] = oracle.dequant_rows(ggml.Q4_K, d[e * db:(e + 1) * db], H, I)
    ref, bd = moe_reference_bf16(x.float().numpy(), rid, rw, Wg, Wu, Wd)
    check_bf16(y, ref, bd, f"config4 bf16 T={T}")
