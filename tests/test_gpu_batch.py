"""GPU parity of the multi-request decode (ming_lm_batch_step over a paged KV
cache) against the oracle and against the batch-1 step.

The batched step has no reference counterpart (the reference serves one
request at a time); per sequence it must be the batch-1 layer
(src/ming_model.zig:566-614).  Checks:
- every layer of every sequence against the oracle run on the GPU's own input
  to that layer and the sequence's contiguous cache (q|k|v, attention, x1,
  swiglu, output, the appended k/v rows read back from the pages), then
  the head on the GPU's stack output: bf16 bar 2e-2 + 1e-2 |ref|, logits
  2e-2 + 1e-2 |ref|, argmax equal where the oracle's top-2 margin > 1e-4;
- sequence i of a batch against ming_lm_step on a contiguous cache with the
  same rows (2-layer model, so the two f32 summation orders do not drift):
  hidden and logits within the same bars;
- the page placement does not matter: a second page table over the same rows
  gives bit-identical hidden, logits and ids;
- positions advance by one; bad positions / page ids report
  MING_E_CTX_OVER_CAPACITY from ming_sync without touching other memory."""
import numpy as np
import pytest
import torch

import oracle
from lmkit import assert_close_bf16, oracle_model

pytestmark = pytest.mark.gpu

MARGIN = 1e-4


def syn_mod(ming):
    import importlib

    return importlib.import_module("ming-tts-serve_amd.synthetic")


def host_u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def run(ming, batch, pk, tokens):
    n = len(tokens)
    spec = pk.spec
    tok = torch.tensor(tokens, dtype=torch.int32, device="cuda")
    hid = torch.empty((n, spec.hidden), dtype=torch.bfloat16, device="cuda")
    lg = torch.empty((n, spec.vocab), dtype=torch.float32, device="cuda")
    am = torch.empty(n, dtype=torch.int32, device="cuda")
    batch.step(pk, pk.table, pk.pos, tokens=tok, hidden=hid, logits=lg, argmax=am)
    batch.ctx.sync()
    return hid, lg, am


def check_teacher_forced(ming, batch, pk, orc, host, lens, tokens, hid, lg, am, tag, seqs=None, only=None):
    """seqs: the sequences whose every layer is checked (default all); only: the sequences
    checked at all (embedding, appended rows, head; default all)."""
    cfg, layers, norm, head = orc
    tr = {k: host_u16(v) for k, v in batch.trace().items()}
    worst = 0.0
    for i in range(len(lens)):
        if only is not None and i not in only:
            continue
        pos = lens[i]
        assert np.array_equal(tr["x"][0, i], oracle.embed(head, tokens[i])), f"{tag} seq {i} embedding"
        gk, gv = pk.gather(i, pos + 1)
        kc, vc = host[i]
        for l, lay in enumerate(layers if seqs is None or i in seqs else []):
            cap = pos + 1
            k_l = np.zeros((cfg.kv_heads, cap, cfg.head_dim), np.uint16)
            v_l = np.zeros_like(k_l)
            k_l[:, :pos] = kc[l]
            v_l[:, :pos] = vc[l]
            x2, t = oracle.lm_layer_step(cfg, lay, tr["x"][l, i], pos, k_l, v_l, trace=True)
            w = f"{tag} seq {i} (pos {pos}) layer {l}"
            assert_close_bf16(tr["qkv"][l, i], t["qkv"], w + " q|k|v")
            assert_close_bf16(tr["att"][l, i], t["att"], w + " attention")
            assert_close_bf16(tr["x1"][l, i], t["x1"], w + " x1")
            assert_close_bf16(tr["hh"][l, i], t["hh"], w + " swiglu")
            worst = max(worst, assert_close_bf16(tr["x"][l + 1, i], x2, w + " output"))
            assert_close_bf16(gk[l, :, pos], k_l[:, pos], w + " appended k")
            assert_close_bf16(gv[l, :, pos], v_l[:, pos], w + " appended v")
            assert np.array_equal(gk[l, :, :pos], kc[l]) and np.array_equal(gv[l, :, :pos], vc[l]), w + " old rows"
        ram, rhid, rlg, _, margin = oracle.lm_head(cfg, norm, head, tr["x"][-1, i])
        assert_close_bf16(host_u16(hid[i]), rhid, f"{tag} seq {i} final hidden")
        g = lg[i].cpu().numpy().astype(np.float64)
        d = np.abs(g - rlg)
        assert (d <= 2e-2 + 1e-2 * np.abs(rlg)).all(), f"{tag} seq {i} logits: max|d| {d.max():.3e}"
        a = int(am[i].item())
        bar = max(MARGIN, 2.0 * d.max())  # a margin above twice the logit error fixes the argmax
        if margin > bar:
            assert a == ram, f"{tag} seq {i}: argmax {a} != {ram} (margin {margin:.3e})"
        else:
            assert rlg[a] >= rlg[ram] - bar
    return worst


SMALL = dict(hidden=128, heads=2, kv_heads=1, head_dim=64, inter=256, vocab=512, n_layers=2)


@pytest.fixture(scope="module")
def small(ming, ctx):
    S = syn_mod(ming)
    spec = S.LmSpec(**SMALL)
    syn = S.SyntheticLm(ctx, spec, seed=21, quant=True, norm_std=0.1)
    m = syn.model()
    b = ming.LmBatch(m, 64, 1024)
    yield S, spec, syn, m, b, oracle_model(syn)
    b.close()
    m.close()


def ragged(n, lo, hi, seed):
    return [int(v) for v in np.random.default_rng(seed).integers(lo, hi + 1, n)]


@pytest.mark.parametrize("lens", [[0, 1, 63, 64, 200, 300], ragged(40, 1, 700, 1), ragged(64, 1, 1000, 2)],
                         ids=["6seq", "40seq", "64seq"])
def test_batch_small_matches_oracle(ming, ctx, small, lens):
    S, spec, syn, m, b, orc = small
    n = len(lens)
    print(f"[batch] small model, {n} sequences, lens {min(lens)}..{max(lens)}", flush=True)
    pk = S.PagedKv(spec, n, 16, spare=3, seed=n)
    host = pk.fill_random(lens, seed=5)
    tokens = [int(t) for t in ming.synth_uniform_i32(6, f"tok{n}", n, spec.vocab)]
    hid, lg, am = run(ming, b, pk, tokens)
    assert pk.pos.cpu().tolist() == [p + 1 for p in lens]
    worst = check_teacher_forced(ming, b, pk, orc, host, lens, tokens, hid, lg, am, f"{n} seqs")
    print(f"[batch] {n} seqs worst layer max|d| {worst:.3e}", flush=True)


def test_batch_equals_single_sequence_steps(ming, ctx, small):
    S, spec, syn, m, b, orc = small
    lens = [5, 64, 129, 255, 256, 511]
    n = len(lens)
    pk = S.PagedKv(spec, n, 8, seed=11)
    host = pk.fill_random(lens, seed=12)
    tokens = [int(t) for t in ming.synth_uniform_i32(13, "tok.single", n, spec.vocab)]
    hid, lg, am = run(ming, b, pk, tokens)
    for i in range(n):
        cache = S.KvCache(spec, lens[i] + 4)
        kc, vc = host[i]
        cache.k[:, :, :lens[i]] = torch.from_numpy(kc.view(np.int16)).cuda().view(torch.bfloat16)
        cache.v[:, :, :lens[i]] = torch.from_numpy(vc.view(np.int16)).cuda().view(torch.bfloat16)
        cache.kv.len = lens[i]
        tok = torch.tensor([tokens[i]], dtype=torch.int32, device="cuda")
        h1 = torch.empty(spec.hidden, dtype=torch.bfloat16, device="cuda")
        l1 = torch.empty(spec.vocab, dtype=torch.float32, device="cuda")
        a1 = torch.empty(1, dtype=torch.int32, device="cuda")
        m.step(cache.kv, token=tok, hidden=h1, logits=l1, argmax=a1)
        ctx.sync()
        assert_close_bf16(host_u16(hid[i]), host_u16(h1), f"seq {i} hidden vs batch-1")
        r = l1.cpu().numpy().astype(np.float64)
        d = np.abs(lg[i].cpu().numpy() - r)
        assert (d <= 2e-2 + 1e-2 * np.abs(r)).all(), f"seq {i} logits vs batch-1: max|d| {d.max():.3e}"
        # the two steps' stack outputs differ by f32 summation order, so their logits by up to
        # d.max(): where the batch-1 margin exceeds twice that, the picks must agree
        top = np.sort(r)[-2:]
        if top[1] - top[0] > 2 * d.max() + MARGIN:
            assert int(am[i].item()) == int(a1.item())
        # the appended rows agree with the batch-1 cache's
        gk, gv = pk.gather(i, lens[i] + 1)
        ck, cv = cache.host()
        assert_close_bf16(gk[:, :, lens[i]], ck[:, :, lens[i]], f"seq {i} appended k vs batch-1")
        assert_close_bf16(gv[:, :, lens[i]], cv[:, :, lens[i]], f"seq {i} appended v vs batch-1")


def test_page_placement_invariance(ming, ctx, small):
    S, spec, syn, m, b, orc = small
    lens = ragged(20, 1, 900, 3)
    n = len(lens)
    tokens = [int(t) for t in ming.synth_uniform_i32(14, "tok.perm", n, spec.vocab)]
    outs = []
    for seed in (1, 2):
        pk = S.PagedKv(spec, n, 16, spare=7, seed=seed)
        pk.fill_random(lens, seed=15)
        outs.append(run(ming, b, pk, tokens))
    for a, c in zip(outs[0], outs[1]):
        assert torch.equal(a, c)


def test_batch_capacity_errors(ming, ctx, small):
    S, spec, syn, m, b, orc = small
    lens = [10, 20]
    pk = S.PagedKv(spec, 2, 2, seed=4)
    pk.fill_random(lens, seed=16)
    pk.pos[1] = 128  # = pages_per_seq * 64: no room
    tok = torch.tensor([1, 2], dtype=torch.int32, device="cuda")
    b.step(pk, pk.table, pk.pos, tokens=tok)
    with pytest.raises(ming.MingError) as e:
        ctx.sync()
    assert e.value.status == ming.MING_E_CTX_OVER_CAPACITY
    pk.pos.copy_(torch.tensor(lens, dtype=torch.int32))
    t = pk.table_host.copy()
    t[0, 0] = pk.n_pages  # out of the pool
    pk.set_table(t)
    b.step(pk, pk.table, pk.pos, tokens=tok)
    with pytest.raises(ming.MingError) as e:
        ctx.sync()
    assert e.value.status == ming.MING_E_CTX_OVER_CAPACITY
    # a clean step afterwards succeeds
    pk.set_table(np.arange(4, dtype=np.int32).reshape(2, 2))
    pk.pos.copy_(torch.tensor(lens, dtype=torch.int32))
    b.step(pk, pk.table, pk.pos, tokens=tok)
    ctx.sync()
    with pytest.raises(ming.MingError) as e:  # pages_per_seq * 64 beyond max_ctx
        b.step(pk, torch.zeros((2, 17), dtype=torch.int32, device="cuda"), pk.pos, tokens=tok)
    assert e.value.status == ming.MING_E_CTX_OVER_CAPACITY


@pytest.fixture(scope="module")
def qwen(ming, ctx):
    S = syn_mod(ming)
    print("[batch] building 24-layer 4-bit Qwen2-0.5B-shaped model", flush=True)
    syn = S.SyntheticLm(ctx, S.QWEN2_05B, seed=0, quant=True)
    m = syn.model()
    b = ming.LmBatch(m, 64, 4096)
    oracle.set_threads(16)
    yield S, syn, m, b, oracle_model(syn)
    b.close()
    m.close()


def test_batch_qwen_shape_matches_oracle(ming, ctx, qwen):
    """16 sequences with contexts in [128, 4096] (every sequence's every layer
    is checked for 4 of them, the head for all)."""
    S, syn, m, b, orc = qwen
    spec = syn.spec
    lens = ragged(16, 128, 4096 - 1, 0)
    print(f"[batch] qwen shape, 16 sequences, lens {lens}", flush=True)
    pk = S.PagedKv(spec, 16, 64, seed=0)
    host = pk.fill_random(lens, seed=0)
    tokens = [int(t) for t in ming.synth_uniform_i32(0, "tok.c5", 16, spec.vocab)]
    hid, lg, am = run(ming, b, pk, tokens)
    order = np.argsort(lens)
    seqs = [int(order[0]), int(order[5]), int(order[10]), int(order[-1])]
    worst = check_teacher_forced(ming, b, pk, orc, host, lens, tokens, hid, lg, am, "qwen", seqs=seqs)
    print(f"[batch] qwen shape worst layer max|d| {worst:.3e}", flush=True)


def test_batch_qwen_shape_64_matches_oracle(ming, ctx, qwen):
    """The multi-request server decode at 64 sequences, contexts uniform in
    [128, 4096]: every layer of 7 sequences spread over the contexts (the
    shortest, the longest and 5 between), the final hidden, logits and argmax
    of all 64."""
    S, syn, m, b, orc = qwen
    spec = syn.spec
    lens = ragged(64, 128, 4096 - 1, 3)
    print(f"[batch] qwen shape, 64 sequences, lens {min(lens)}..{max(lens)}", flush=True)
    pk = S.PagedKv(spec, 64, 64, seed=3)
    host = pk.fill_random(lens, seed=3)
    tokens = [int(t) for t in ming.synth_uniform_i32(3, "tok.c5.64", 64, spec.vocab)]
    hid, lg, am = run(ming, b, pk, tokens)
    order = np.argsort(lens)
    seqs = [int(order[j]) for j in (0, 10, 21, 32, 43, 53, 63)]
    worst = check_teacher_forced(ming, b, pk, orc, host, lens, tokens, hid, lg, am, "qwen64", seqs=seqs)
    print(f"[batch] qwen shape 64 sequences worst layer max|d| {worst:.3e}", flush=True)


def test_batch_step_beyond_64_sequences(ming, ctx, qwen):
    """The batched step above 64 sequences (a batch of 512 rows: the LDS-tiled GEMMs, the tiled
    head with 64-column argmax partials, paged attention and merge beyond 64 sequences): 65
    sequences in one call equal the same sequences as calls of 64 and 1, bit for bit (hidden,
    logits, ids, cache rows); 512 sequences with short ragged contexts match the oracle, every
    layer of 3 of them and the head of 10."""
    S, syn, m, b, orc = qwen
    spec = syn.spec
    big = ming.LmBatch(m, 512, 1024)
    try:
        lens = ragged(65, 1, 300, 5)
        tokens = [int(t) for t in ming.synth_uniform_i32(5, "tok.c5.65", 65, spec.vocab)]
        tok = torch.tensor(tokens, dtype=torch.int32, device="cuda")
        print(f"[batch] 65 sequences in one call vs 64 + 1, lens {min(lens)}..{max(lens)}", flush=True)
        outs = []
        for split in (False, True):
            pk = S.PagedKv(spec, 65, 5, seed=5)
            pk.fill_random(lens, seed=5)
            hid = torch.empty((65, spec.hidden), dtype=torch.bfloat16, device="cuda")
            lg = torch.empty((65, spec.vocab), dtype=torch.float32, device="cuda")
            am = torch.empty(65, dtype=torch.int32, device="cuda")
            if not split:
                big.step(pk, pk.table, pk.pos, tokens=tok, hidden=hid, logits=lg, argmax=am)
            else:
                for lo, hi in ((0, 64), (64, 65)):
                    b.step(pk, pk.table[lo:hi], pk.pos[lo:hi], tokens=tok[lo:hi], hidden=hid[lo:hi],
                           logits=lg[lo:hi], argmax=am[lo:hi])
            ctx.sync()
            outs.append((hid, lg, am, pk.gather(64, lens[64] + 1), pk.gather(0, lens[0] + 1)))
        (h0, l0, a0, c0, d0), (h1, l1, a1, c1, d1) = outs
        assert torch.equal(h0, h1), "hidden differs between one call of 65 and calls of 64 + 1"
        assert torch.equal(l0, l1), "logits differ between one call of 65 and calls of 64 + 1"
        assert torch.equal(a0, a1), "ids differ between one call of 65 and calls of 64 + 1"
        for x, y in ((c0, c1), (d0, d1)):
            assert np.array_equal(x[0], y[0]) and np.array_equal(x[1], y[1]), "cache rows differ"
        del outs, l0, l1
        n = 512
        lens = ragged(n, 1, 120, 6)
        print(f"[batch] 512 sequences, lens {min(lens)}..{max(lens)}", flush=True)
        pk = S.PagedKv(spec, n, 2, seed=6)
        host = pk.fill_random(lens, seed=6)
        tokens = [int(t) for t in ming.synth_uniform_i32(6, "tok.c5.512", n, spec.vocab)]
        hid, lg, am = run(ming, big, pk, tokens)
        order = np.argsort(lens)
        seqs = [int(order[0]), int(order[255]), int(order[-1])]
        only = set(seqs) | {0, 63, 64, 65, 127, 128, 300, 511}
        worst = check_teacher_forced(ming, big, pk, orc, host, lens, tokens, hid, lg, am, "qwen512", seqs=seqs,
                                     only=only)
        print(f"[batch] 512 sequences worst layer max|d| {worst:.3e}", flush=True)
    finally:
        big.close()


# ---- multi-token prefill (rows of one sequence as sequences sharing its pages) ----

def one_row_table(pk):
    return pk.table[0].contiguous()


def test_prefill_equals_single_row_steps(ming, ctx, small):
    """70 prompt rows after 10 cached ones (a 64-row chunk and a 6-row chunk):
    hidden rows, logits, ids and the cache equal 70 one-row steps bit for bit."""
    S, spec, syn, m, b, orc = small
    L, pos0 = 70, 10
    toks = ming.synth_uniform_i32(31, "prefill.tok", L, spec.vocab)
    tok = torch.tensor([int(t) for t in toks], dtype=torch.int32, device="cuda")
    outs = []
    for mode in ("prefill", "steps"):
        pk = S.PagedKv(spec, 1, 2, spare=5, seed=3)
        pk.fill_random([pos0], seed=32)
        hid = torch.empty((L, spec.hidden), dtype=torch.bfloat16, device="cuda")
        lg = torch.empty((L, spec.vocab), dtype=torch.float32, device="cuda")
        am = torch.empty(L, dtype=torch.int32, device="cuda")
        if mode == "prefill":
            b.prefill(pk, one_row_table(pk), pos0, tokens=tok, hidden=hid, logits=lg, argmax=am)
        else:
            pos = torch.empty(1, dtype=torch.int32, device="cuda")
            for i in range(L):
                pos.fill_(pos0 + i)
                b.step(pk, pk.table, pos, tokens=tok[i:i + 1], hidden=hid[i:i + 1], logits=lg[i:i + 1],
                       argmax=am[i:i + 1])
        ctx.sync()
        outs.append((hid, lg, am, pk.gather(0, pos0 + L)))
    (h0, l0, a0, (k0, v0)), (h1, l1, a1, (k1, v1)) = outs
    assert torch.equal(h0, h1) and torch.equal(l0, l1) and torch.equal(a0, a1)
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)


def test_prefill_matches_oracle(ming, ctx, small):
    """20 prompt rows from position 0: every layer of every row against the
    oracle on the GPU's own layer input and the rows the GPU cached before it."""
    S, spec, syn, m, b, orc = small
    cfg, layers, norm, head = orc
    L = 20
    pk = S.PagedKv(spec, 1, 1, spare=2, seed=5)
    x = ming.synth_normal_bf16(33, "prefill.x", L * spec.hidden).reshape(L, spec.hidden)
    hid = torch.empty((L, spec.hidden), dtype=torch.bfloat16, device="cuda")
    b.prefill(pk, one_row_table(pk), 0, x_in=torch.from_numpy(x.view(np.int16)).cuda().view(torch.bfloat16),
              hidden=hid)
    ctx.sync()
    tr = {k: host_u16(v) for k, v in b.trace().items()}
    gk, gv = pk.gather(0, L)
    assert np.array_equal(tr["x"][0], x)
    for i in range(L):
        for l, lay in enumerate(layers):
            k_l = np.zeros((cfg.kv_heads, i + 1, cfg.head_dim), np.uint16)
            v_l = np.zeros_like(k_l)
            k_l[:, :i] = gk[l, :, :i]
            v_l[:, :i] = gv[l, :, :i]
            x2, t = oracle.lm_layer_step(cfg, lay, tr["x"][l, i], i, k_l, v_l, trace=True)
            w = f"prefill row {i} layer {l}"
            assert_close_bf16(tr["qkv"][l, i], t["qkv"], w + " q|k|v")
            assert_close_bf16(tr["att"][l, i], t["att"], w + " attention (causal)")
            assert_close_bf16(tr["x"][l + 1, i], x2, w + " output")
            assert_close_bf16(gk[l, :, i], k_l[:, i], w + " cached k")
            assert_close_bf16(gv[l, :, i], v_l[:, i], w + " cached v")
        _, rhid, _, _, _ = oracle.lm_head(cfg, norm, head, tr["x"][-1, i])
        assert_close_bf16(host_u16(hid[i]), rhid, f"prefill row {i} hidden")


def test_prefill_512_row_chunk_equals_64_row_chunks(ming, ctx, qwen):
    """The Qwen shape: a 300-row prompt after 40 cached rows through a batch of
    512 rows (one chunk: every GEMM call has 300 rows) equals the same prompt
    through 64-row chunks bit for bit -- hidden rows, the cache, logits and
    ids (a GEMM of more than 64 rows splits K exactly as one of <= 64 rows) -- and 4 rows
    spread over the prompt match the oracle layer by layer on their own inputs
    and the rows cached before them."""
    S, syn, m, b64, orc = qwen
    spec = syn.spec
    cfg, layers, norm, head = orc
    L, pos0 = 300, 40
    print(f"[prefill] qwen shape, {L} rows after {pos0}: one 512-row chunk vs 64-row chunks", flush=True)
    big = ming.LmBatch(m, 512, 1024)
    x = ming.synth_normal_bf16(35, "prefill.big.x", L * spec.hidden).reshape(L, spec.hidden)
    xd = torch.from_numpy(x.view(np.int16)).cuda().view(torch.bfloat16)
    outs = []
    for bt in (big, b64):
        pk = S.PagedKv(spec, 1, 6, spare=2, seed=9)
        pk.fill_random([pos0], seed=36)
        hid = torch.empty((L, spec.hidden), dtype=torch.bfloat16, device="cuda")
        lg = torch.empty((L, spec.vocab), dtype=torch.float32, device="cuda")
        am = torch.empty(L, dtype=torch.int32, device="cuda")
        bt.prefill(pk, one_row_table(pk), pos0, x_in=xd, hidden=hid, logits=lg, argmax=am)
        ctx.sync()
        outs.append((hid, pk.gather(0, pos0 + L), lg, am))
    (h0, (k0, v0), lg0, am0), (h1, (k1, v1), lg1, am1) = outs
    assert torch.equal(h0, h1), "hidden rows differ between 512-row and 64-row chunks"
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1), "cache rows differ"
    # the head of a 300-row call (the tiled GEMM) and of <= 64-row calls (the LDS-resident head
    # kernel, 32-column argmax partials) give the same logits and ids
    assert torch.equal(lg0, lg1), "logits differ between the head launches for 300 and 64 rows"
    assert torch.equal(am0, am1), "argmax differs between the head launches for 300 and 64 rows"
    del lg0, lg1
    tr = {k: host_u16(v) for k, v in big.trace().items()}
    big.close()
    for i in (0, 99, 199, 299):
        p = pos0 + i
        for l, lay in enumerate(layers):
            k_l = np.zeros((cfg.kv_heads, p + 1, cfg.head_dim), np.uint16)
            v_l = np.zeros_like(k_l)
            k_l[:, :p] = k0[l, :, :p]
            v_l[:, :p] = v0[l, :, :p]
            x2, t = oracle.lm_layer_step(cfg, lay, tr["x"][l, i], p, k_l, v_l, trace=True)
            w = f"prefill row {i} (pos {p}) layer {l}"
            assert_close_bf16(tr["qkv"][l, i], t["qkv"], w + " q|k|v")
            assert_close_bf16(tr["att"][l, i], t["att"], w + " attention (causal)")
            assert_close_bf16(tr["x1"][l, i], t["x1"], w + " x1")
            assert_close_bf16(tr["hh"][l, i], t["hh"], w + " swiglu")
            assert_close_bf16(tr["x"][l + 1, i], x2, w + " output")
            assert_close_bf16(k0[l, :, p], k_l[:, p], w + " cached k")
            assert_close_bf16(v0[l, :, p], v_l[:, p], w + " cached v")
        _, rhid, _, _, _ = oracle.lm_head(cfg, norm, head, tr["x"][-1, i])
        assert_close_bf16(host_u16(h0[i]), rhid, f"prefill row {i} hidden")


def test_prefill_capacity_error(ming, ctx, small):
    S, spec, syn, m, b, orc = small
    pk = S.PagedKv(spec, 1, 1, seed=6)
    tok = torch.zeros(10, dtype=torch.int32, device="cuda")
    with pytest.raises(ming.MingError) as e:
        b.prefill(pk, one_row_table(pk), 60, tokens=tok)  # 60 + 10 > 64
    assert e.value.status == ming.MING_E_CTX_OVER_CAPACITY
