"""gfx950 packed variable-length attention (sage_forward_varlen, cdna4_sage.attention_varlen, sageattn_varlen).

The reference runs one sageattn call per sequence (src/sageattention/core.py:80-88).  The native pass must give, for
every sequence, exactly what a separate call on that sequence gives: the same intermediates (Q8 / QS rows, K8 / KS /
V8T rows at the sequence's padded offset, VS) and the same output, bit for bit, against the unsplit sage_forward
(workspace NULL: every query tile whole, as in the varlen pass).  Sequences a separate call cannot run (causal with
q_len > kv_len, no keys) are checked against the CPU oracle's per-sequence restatement."""
import os

import numpy as np
import pytest
import torch

import cdna4_sage
import sageattention
from cdna4_sage import _capi
from gpu_util import DT, cosine, stream
from oracle import sage_oracle as orc

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2   # vs the oracle's emulation with the reference's 32-key rescale blocks
COS = 0.999      # vs float64 attention


def _packed(lq, lk, H, Hkv, D, dt, seed, extra_q=0):
    g = torch.Generator().manual_seed(seed)
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    q = torch.randn(int(cu_q[-1]) + extra_q, H, D, generator=g).to(dt)
    k = torch.randn(int(cu_k[-1]), Hkv, D, generator=g).to(dt)
    v = torch.randn(int(cu_k[-1]), Hkv, D, generator=g).to(dt)
    return q, k, v, cu_q, cu_k


def _varlen_capi(q, k, v, cu_q, cu_k, causal, out=None):
    """sage_forward_varlen on device tensors; returns the output and every intermediate (device tensors)."""
    dev = q.device
    TQ, H, D = q.shape
    TK, Hkv = k.shape[0], k.shape[1]
    batch = len(cu_q) - 1
    tkp, wsb = _capi.varlen_layout(batch, H, Hkv, TQ, TK)
    dl = _capi.layout_dim(D)
    r = dict(q8=torch.empty(H, TQ, dl, dtype=torch.int8, device=dev),
             qs=torch.empty(H, TQ, dtype=torch.float32, device=dev),
             k8=torch.empty(Hkv, tkp, dl, dtype=torch.int8, device=dev),
             ks=torch.empty(Hkv, tkp // 32, dtype=torch.float32, device=dev),
             v8t=torch.empty(Hkv, dl, tkp, dtype=torch.uint8, device=dev),
             vs=torch.empty(batch, Hkv, dl, dtype=torch.float32, device=dev),
             ws=torch.empty(wsb, dtype=torch.uint8, device=dev),
             out=torch.empty(TQ, H, D, dtype=q.dtype, device=dev) if out is None else out)
    cq = torch.tensor(cu_q, dtype=torch.int32, device=dev)
    ck = torch.tensor(cu_k, dtype=torch.int32, device=dev)
    _capi.call("sage_forward_varlen", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
               v.data_ptr(), v.stride(0), v.stride(1), r["out"].data_ptr(), r["out"].stride(0), r["out"].stride(1),
               cq.data_ptr(), ck.data_ptr(), batch, H, Hkv, TQ, TK, D, DT[q.dtype], int(causal), 1.0,
               r["q8"].data_ptr(), r["qs"].data_ptr(), r["k8"].data_ptr(), r["ks"].data_ptr(), r["v8t"].data_ptr(),
               r["vs"].data_ptr(), r["ws"].data_ptr(), wsb, stream(dev))
    torch.cuda.synchronize(dev)
    return r


def _dense_capi(qi, ki, vi, causal):
    """One sequence through sage_forward without a workspace (unsplit tiles): NHD views [S, heads, D] as B = 1."""
    dev = qi.device
    Sq, H, D = qi.shape
    Skv, Hkv = ki.shape[0], ki.shape[1]
    skp = _capi.kv_pad(Skv)
    dl = _capi.layout_dim(D)
    r = dict(q8=torch.empty(1, H, Sq, dl, dtype=torch.int8, device=dev),
             qs=torch.empty(1, H, Sq, dtype=torch.float32, device=dev),
             k8=torch.empty(1, Hkv, skp, dl, dtype=torch.int8, device=dev),
             ks=torch.empty(1, Hkv, skp // 32, dtype=torch.float32, device=dev),
             v8t=torch.empty(1, Hkv, dl, skp, dtype=torch.uint8, device=dev),
             vs=torch.empty(1, Hkv, dl, dtype=torch.float32, device=dev),
             out=torch.empty(1, Sq, H, D, dtype=qi.dtype, device=dev))
    o = r["out"]
    _capi.call("sage_forward", qi.data_ptr(), 0, qi.stride(0), qi.stride(1), ki.data_ptr(), 0, ki.stride(0),
               ki.stride(1), vi.data_ptr(), 0, vi.stride(0), vi.stride(1), o.data_ptr(), 0, o.stride(1), o.stride(2),
               1, H, Hkv, Sq, Skv, D, DT[qi.dtype], int(causal), 1.0, r["q8"].data_ptr(), r["qs"].data_ptr(),
               r["k8"].data_ptr(), r["ks"].data_ptr(), r["v8t"].data_ptr(), r["vs"].data_ptr(), None, 0, stream(dev))
    torch.cuda.synchronize(dev)
    return r


def _pad128(n):
    return (n + 127) // 128 * 128


def _check_against_separate_calls(q, k, v, cu_q, cu_k, causal, r):
    """Every sequence a separate sage_forward can run: intermediates and output bit for bit."""
    kp = 0
    checked = 0
    for i in range(len(cu_q) - 1):
        q0, q1, k0, k1 = (int(x) for x in (cu_q[i], cu_q[i + 1], cu_k[i], cu_k[i + 1]))
        n = k1 - k0
        if q1 > q0 and n > 0 and not (causal and q1 - q0 > n):
            d = _dense_capi(q[q0:q1], k[k0:k1], v[k0:k1], causal)
            skp = _pad128(n)
            assert torch.equal(r["q8"][:, q0:q1], d["q8"][0]), i
            assert torch.equal(r["qs"][:, q0:q1], d["qs"][0]), i
            assert torch.equal(r["k8"][:, kp:kp + skp], d["k8"][0]), i
            assert torch.equal(r["ks"][:, kp // 32:(kp + skp) // 32], d["ks"][0]), i
            assert torch.equal(r["v8t"][:, :, kp:kp + skp], d["v8t"][0]), i
            assert torch.equal(r["vs"][i], d["vs"][0]), i
            assert torch.equal(r["out"][q0:q1], d["out"][0]), i
            checked += 1
        kp += _pad128(n)
    return checked


def _check_against_oracle(q, k, v, cu_q, cu_k, causal, out, out_dtype):
    emu = orc.sage_forward_varlen(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu_q, cu_k,
                                  causal=causal, block_n=32, out_dtype=out_dtype)
    got = out.float().cpu().numpy()
    rows = ~np.isnan(emu[:, 0, 0])
    assert float(np.abs(got[rows] - emu[rows]).max()) <= MAX_ABS
    hnd = lambda t: np.ascontiguousarray(t.transpose(1, 0, 2))[None]   # noqa: E731
    for i in range(len(cu_q) - 1):
        q0, q1, k0, k1 = (int(x) for x in (cu_q[i], cu_q[i + 1], cu_k[i], cu_k[i + 1]))
        if q1 == q0:
            continue
        if k1 == k0:
            assert (got[q0:q1] == 0).all()
            continue
        off = max(0, (q1 - q0) - (k1 - k0)) if causal else 0      # causal rows that see no key are 0
        assert (got[q0:q0 + off] == 0).all()
        if q1 - q0 - off < 2:
            continue
        ref = orc.sdpa_reference(hnd(q[q0 + off:q1].float().numpy()), hnd(k[k0:k1].float().numpy()),
                                 hnd(v[k0:k1].float().numpy()), causal=causal)[0].transpose(1, 0, 2)
        assert cosine(got[q0 + off:q1], ref) >= COS, i


VARLEN_CASES = [  # lq, lk, H, Hkv, D, dtype, causal
    ([300, 1, 700, 129, 0, 64], [300, 1000, 700, 77, 50, 64], 4, 2, 128, torch.bfloat16, False),
    ([257, 100, 40, 513], [257, 300, 20, 513], 4, 1, 64, torch.float16, True),     # sequence 2: q_len > kv_len
    ([64, 200, 33], [128, 0, 1000], 2, 2, 128, torch.bfloat16, True),            # sequence 1 has no keys
    ([1000, 3, 1], [1000, 3, 1], 8, 8, 64, torch.bfloat16, False),
    ([300, 90, 700], [500, 90, 650], 4, 2, 96, torch.bfloat16, True),
    ([200, 333], [260, 700], 2, 1, 256, torch.float16, False),
    ([100, 300], [0, 500], 4, 2, 128, torch.bfloat16, False),                    # sequence 0 (first rows) has no keys
    ([70, 130, 200], [0, 0, 300], 2, 1, 64, torch.float16, True),
]


@pytest.mark.parametrize("lq,lk,H,Hkv,D,dt,causal", VARLEN_CASES)
def test_varlen_matches_separate_calls_and_oracle(dev, lq, lk, H, Hkv, D, dt, causal):
    q, k, v, cu_q, cu_k = _packed(lq, lk, H, Hkv, D, dt, seed=sum(lq) + 7 * sum(lk))
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    r = _varlen_capi(qd, kd, vd, cu_q, cu_k, causal)
    assert int(r["ws"][:4].view(torch.int32)[0]) == 0
    assert _check_against_separate_calls(qd, kd, vd, cu_q, cu_k, causal, r) >= 1
    _check_against_oracle(q, k, v, cu_q, cu_k, causal, r["out"], "bf16" if dt == torch.bfloat16 else "f16")


def test_varlen_rows_outside_sequences_and_invalid_cu_seqlens(dev):
    q, k, v, cu_q, cu_k = _packed([100, 200], [300, 50], 4, 2, 128, torch.bfloat16, seed=3, extra_q=40)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    sentinel = torch.full((q.shape[0], 4, 128), 7.0, dtype=torch.bfloat16, device=dev)
    r = _varlen_capi(qd, kd, vd, cu_q, cu_k, False, out=sentinel.clone())
    assert (r["out"][300:] == 7.0).all() and not (r["out"][:300] == 7.0).any()
    # cu_seqlens past the packed totals or decreasing: nothing written, flag set in the workspace
    for bad_q, bad_k in (([0, 100, 400], [0, 300, 350]), ([0, 100, 300], [0, 300, 200]), ([0, 150, 100], [0, 1, 2])):
        r = _varlen_capi(qd, kd, vd, np.array(bad_q, np.int32), np.array(bad_k, np.int32), True,
                         out=sentinel.clone())
        assert (r["out"] == 7.0).all()
        assert int(r["ws"][:4].view(torch.int32)[0]) == 1


def test_varlen_python_api_and_router(dev):
    lq, lk = [1500, 700, 0, 2100], [1500, 1200, 64, 2100]
    q, k, v, cu_q, cu_k = _packed(lq, lk, 8, 2, 128, torch.float16, seed=11)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    cq, ck = torch.tensor(cu_q, device=dev), torch.tensor(cu_k.astype(np.int64), device=dev)   # int32 and int64
    out = cdna4_sage.attention_varlen(qd, kd, vd, cq, ck, max(lq), max(lk), is_causal=True)
    r = _varlen_capi(qd, kd, vd, cu_q, cu_k, True)
    assert torch.equal(out[:4300], r["out"][:4300])
    # the reference's route for each sequence: with 8 heads none of these reaches MIN_WORK (1500^2 * 8 / 2 < 64 Mi), so
    # sageattn_varlen gives what one sageattn call per sequence gives (SDPA here), as the reference's host loop does
    routed = sageattention.sageattn_varlen(qd, kd, vd, cq, ck, max(lq), max(lk), is_causal=True)
    for (q0, q1), (k0, k1) in zip(zip(cu_q[:-1], cu_q[1:]), zip(cu_k[:-1], cu_k[1:])):
        if q1 > q0:
            one = sageattention.sageattn(qd[q0:q1].unsqueeze(0), kd[k0:k1].unsqueeze(0), vd[k0:k1].unsqueeze(0),
                                         tensor_layout="NHD", is_causal=True)[0]
            assert torch.equal(routed[q0:q1], one)
    # without the per-sequence route (CDNA4_SAGE_VARLEN_ROUTE=0) every sequence runs the packed pass, unsynchronised
    import cdna4_sage as cs
    saved = cs.VARLEN_ROUTE
    try:
        cs.VARLEN_ROUTE = False
        assert torch.equal(sageattention.sageattn_varlen(qd, kd, vd, cq, ck, max(lq), max(lk), is_causal=True), out)
    finally:
        cs.VARLEN_ROUTE = saved
    # sm_scale folds into the Q scales as in the dense path: sequence 0 against float32 attention at that scale
    o2 = cdna4_sage.attention_varlen(qd, kd, vd, cq, ck, sm_scale=0.05)
    q0 = qd[:1500].transpose(0, 1).float().contiguous()                               # [8, 1500, 128]
    kt = kd[:1500].float().repeat_interleave(4, 1).permute(1, 2, 0).contiguous()      # [8, 128, 1500]
    v0 = vd[:1500].float().repeat_interleave(4, 1).transpose(0, 1).contiguous()       # [8, 1500, 128]
    ref = torch.softmax(torch.matmul(q0, kt) * 0.05, dim=-1).matmul(v0)
    assert cosine(o2[:1500].float().cpu().numpy(), ref.transpose(0, 1).cpu().numpy()) >= COS
    # a scale that is not positive selects the default 1/sqrt(D), as the reference's op does for its per-sequence calls
    # (it used to fold into the Q scales as 0 or a negative factor)
    for sm in (0.0, -0.05, float("nan")):
        o3 = cdna4_sage.attention_varlen(qd, kd, vd, cq, ck, max(lq), max(lk), sm_scale=sm, is_causal=True)
        assert torch.equal(o3[:4300], out[:4300])
    # all sequences shorter than the kernel's minimum key length: the reference's per-sequence routing (SDPA here)
    q, k, v, cu_q, cu_k = _packed([100, 300], [200, 300], 4, 4, 64, torch.bfloat16, seed=12)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    small = sageattention.sageattn_varlen(qd, kd, vd, torch.tensor(cu_q, device=dev), torch.tensor(cu_k, device=dev),
                                          300, 300)
    for (q0, q1, k0, k1) in ((0, 100, 0, 200), (100, 400, 200, 500)):
        ref = torch.nn.functional.scaled_dot_product_attention(
            qd[q0:q1].transpose(0, 1).float(), kd[k0:k1].transpose(0, 1).float(), vd[k0:k1].transpose(0, 1).float())
        torch.testing.assert_close(small[q0:q1].float(), ref.transpose(0, 1), atol=2e-2, rtol=0)


def test_varlen_routes_each_sequence_like_the_reference(dev):
    """A batch whose sequences take both routes of the reference's per-sequence sageattn calls
    (src/sageattention/core.py:80-88): sequences 0 and 2 reach MIN_KV and MIN_WORK with 8 heads and run the packed
    kernel pass (bit-equal to the pass on the whole batch), sequence 1 (500 keys) and the causal sequence longer than
    its keys go to sageattn alone (torch SDPA, exact), an empty query sequence is skipped."""
    for causal, lq, lk in ((False, [3000, 500, 0, 2900], [3000, 500, 40, 2900]),
                           (True, [4200, 900, 4300], [4200, 600, 4300])):
        q, k, v, cu_q, cu_k = _packed(lq, lk, 8, 4, 128, torch.bfloat16, seed=31 + causal)
        qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
        cq, ck = torch.tensor(cu_q, device=dev), torch.tensor(cu_k, device=dev)
        routed = sageattention.sageattn_varlen(qd, kd, vd, cq, ck, max(lq), max(lk), is_causal=causal)
        packed = cdna4_sage.attention_varlen(qd, kd, vd, cq, ck, max(lq), max(lk), is_causal=causal)
        kinds = []
        for (q0, q1), (k0, k1) in zip(zip(cu_q[:-1], cu_q[1:]), zip(cu_k[:-1], cu_k[1:])):
            if q1 == q0:
                continue
            work = 8 * (q1 - q0) * (k1 - k0) // (2 if causal else 1)
            kernel = (k1 - k0) >= cdna4_sage.MIN_KV and work >= cdna4_sage.MIN_WORK and not (causal and q1 - q0 > k1 - k0)
            kinds.append(kernel)
            if kernel:
                assert torch.equal(routed[q0:q1], packed[q0:q1])
            else:
                ref = torch.nn.functional.scaled_dot_product_attention(
                    qd[q0:q1].transpose(0, 1)[None], kd[k0:k1].transpose(0, 1)[None], vd[k0:k1].transpose(0, 1)[None],
                    is_causal=False, enable_gqa=True,
                    attn_mask=(torch.ones(q1 - q0, k1 - k0, dtype=torch.bool, device=dev).tril(int(k1 - k0) - int(q1 - q0))
                               if causal else None))
                torch.testing.assert_close(routed[q0:q1].float(), ref[0].transpose(0, 1).float(), atol=1e-2, rtol=0)
                assert not torch.equal(routed[q0:q1], packed[q0:q1])
        assert any(kinds) and not all(kinds), kinds


def test_varlen_mixed_lengths_at_scale(dev):
    """A packed batch of Flux-like and short sequences (24 heads, head_dim 128): every sequence bit-exact against
    its own call; prints the packed pass against the per-sequence calls."""
    lq = [4608, 1000, 3000, 128, 2500, 700]
    q, k, v, cu_q, cu_k = _packed(lq, lq, 24, 24, 128, torch.bfloat16, seed=13)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    r = _varlen_capi(qd, kd, vd, cu_q, cu_k, False)
    assert _check_against_separate_calls(qd, kd, vd, cu_q, cu_k, False, r) == len(lq)
    cq, ck = torch.tensor(cu_q, device=dev), torch.tensor(cu_k, device=dev)
    f_var = lambda: cdna4_sage.attention_varlen(qd, kd, vd, cq, ck, max(lq), max(lq))   # noqa: E731
    f_seq = lambda: [cdna4_sage.attention(qd[a:b].unsqueeze(0), kd[a:b].unsqueeze(0), vd[a:b].unsqueeze(0), "NHD")  # noqa: E731
                     for a, b in zip(cu_q[:-1], cu_q[1:])]
    ms = {}
    for name, f in (("packed", f_var), ("per-sequence", f_seq)):
        for _ in range(3):
            f()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            f()
        e1.record()
        torch.cuda.synchronize(dev)
        ms[name] = e0.elapsed_time(e1) / 10
    print(f"varlen 6 sequences (sum {sum(lq)} tokens, 24 heads, d128): packed {ms['packed']:.3f} ms, "
          f"per-sequence calls {ms['per-sequence']:.3f} ms")


def _random_varlen_cases(n=12, seed=4242):
    rng = np.random.RandomState(seed)
    out = []
    for i in range(n):
        batch = int(rng.randint(1, 7))
        lk = [int(rng.choice([0, int(rng.randint(1, 70)), int(rng.randint(70, 900))], p=[0.1, 0.3, 0.6]))
              for _ in range(batch)]
        causal = bool(rng.rand() < 0.5)
        lq = [int(rng.choice([0, int(rng.randint(1, 64)), int(rng.randint(64, 700))], p=[0.1, 0.3, 0.6]))
              for _ in range(batch)]
        D = int(rng.choice([64, 96, 128, 256]))
        Hkv = int(rng.randint(1, 3))
        H = Hkv * int(rng.choice([1, 2, 4]))
        dt = torch.bfloat16 if rng.rand() < 0.6 else torch.float16
        out.append((i, lq, lk, H, Hkv, D, dt, causal))
    return out


RANDOM_VARLEN = _random_varlen_cases(seed=4242 + int(os.environ.get("SAGE_SWEEP_SEED", "0")))


@pytest.mark.parametrize("case", RANDOM_VARLEN, ids=[f"{c[0]}-b{len(c[1])}-d{c[5]}-H{c[3]}/{c[4]}"
                                                      f"{'-causal' if c[7] else ''}" for c in RANDOM_VARLEN])
def test_varlen_random_batches(dev, case):
    """Seeded random packed batches (1-6 sequences; empty query sequences, sequences without keys, causal sequences
    longer than their keys, GQA, head dims 64-256): every sequence a separate call can run is bit-equal to it, and
    the whole pass is within the emulation's gate."""
    i, lq, lk, H, Hkv, D, dt, causal = case
    if sum(lq) == 0 or sum(lk) == 0:
        lq[0], lk[0] = max(lq[0], 5), max(lk[0], 7)   # the packed totals must be positive
    q, k, v, cu_q, cu_k = _packed(lq, lk, H, Hkv, D, dt, seed=9000 + i)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    r = _varlen_capi(qd, kd, vd, cu_q, cu_k, causal)
    assert int(r["ws"][:4].view(torch.int32)[0]) == 0
    _check_against_separate_calls(qd, kd, vd, cu_q, cu_k, causal, r)
    _check_against_oracle(q, k, v, cu_q, cu_k, causal, r["out"], "bf16" if dt == torch.bfloat16 else "f16")
