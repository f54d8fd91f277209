"""Branch sessions of the HIP forwarder against the oracle.

Mirrors nativeBranches (mlx_branches.go:14-182): suffixes that borrow a
resident prefix read-only, one token per branch per Forward, the shared
prefix and the branch's own suffix under one softmax (branchAttention,
mlx_branches.go:98-114). The library adds private suffixes of different
lengths per branch (append).

The oracle replays every branch in turn on one model prefilled with the
prefix: forward at position P + s rewrites only positions >= P, and
attention at position t reads positions [0, t], so each replay sees the
shared prefix and its own suffix only.
"""
import numpy as np
import pytest

from tinyoai_amd import weights as W

pytestmark = pytest.mark.gpu
HELLO_ABC = [2, 340, 328, 331]


@pytest.fixture(scope="module")
def hip():
    from tinyoai_amd import hip as H
    H.lib()
    return H


def oracle_branches(oracle, config, tensors, prefix_ids, suffixes, steps, half):
    """Per branch: the logits after its suffix, then after each of `steps`
    - 1 greedy tokens (the oracle's own choices), [branch][step][vocab], and
    those tokens [branch][step]."""
    P = len(prefix_ids)
    m = oracle.StableLM(config, tensors, half_kv=half,
                        capacity=P + max(len(s) for s in suffixes) + steps + 1)
    if P:
        m.prefill(np.asarray(prefix_ids, np.int32), 0)
    logits = np.zeros((len(suffixes), steps, config["vocab_size"]), np.float32)
    toks = np.zeros((len(suffixes), steps), np.int32)
    for j, suf in enumerate(suffixes):
        for i, tok in enumerate(suf):
            lg = m.forward(int(tok), P + i, i + 1 == len(suf))
        for s in range(steps):
            logits[j, s] = lg
            toks[j, s] = int(np.argmax(lg))
            if s + 1 < steps:
                lg = m.forward(int(toks[j, s]), P + len(suf) + s)
    m.close()
    return logits, toks


def check_rows(got, want, tag, tol=1e-3):
    for j in range(want.shape[0]):
        span = float(np.ptp(want[j]))
        assert np.max(np.abs(got[j] - want[j])) <= tol * span, (tag, j)
        assert int(np.argmax(got[j])) == int(np.argmax(want[j])), (tag, j)


def branch_case(hip, oracle, config, tensors, resident, prefix, suffixes, steps, kv_bits, append):
    """A forwarder holding `resident` opens len(suffixes) branches at
    `prefix`; each branch takes its suffix (append, or forward when every
    suffix is one token), then steps - 1 lockstep tokens fed from the
    oracle's greedy choices. Logits within 1e-3 of their range of the
    oracle's, identical argmax; the model refuses to change while the
    session is open and continues unchanged after it closes."""
    half = kv_bits == 16
    want, toks = oracle_branches(oracle, config, tensors, resident[:prefix], suffixes, steps, half)
    f = hip.StableLMForwarder(config, tensors)
    f.set_kv_bits(kv_bits)
    f.forward(0, resident, want_logits=False)
    br = f.new_branches(prefix, len(suffixes))
    if append:
        got = br.append(suffixes)
    else:
        got = br.forward([s[0] for s in suffixes])
    assert got.shape == (len(suffixes), config["vocab_size"])
    check_rows(got, want[:, 0], "suffix")
    for name, call in [("forward", lambda: f.forward(len(resident), [1])), ("reset", f.reset),
                       ("kv_bits", lambda: f.set_kv_bits(48 - kv_bits)), ("limit", lambda: f.limit_cache(8)),
                       ("close", lambda: hip.check(hip.lib().tinyoai_stablelm_close(f.h)))]:
        with pytest.raises(hip.TinyoaiError, match="branch session"):
            call()
    for s in range(1, steps):
        got = br.forward(toks[:, s - 1])
        check_rows(got, want[:, s], f"step {s}")
    for j, suf in enumerate(suffixes):
        assert br.length(j) == len(suf) + steps - 1
    br.close()
    with pytest.raises(hip.TinyoaiError):
        br.forward(toks[:, 0])  # closed
    with pytest.raises(hip.TinyoaiError):
        f.new_branches(len(resident) + 1, 2)  # beyond the resident prefix
    # the model continues as if no branch had run
    ref = oracle.StableLM(config, tensors, half_kv=half, capacity=len(resident) + 2)
    ref.prefill(np.asarray(resident, np.int32), 0)
    w = ref.forward(7, len(resident))
    g = f.forward(len(resident), [7])
    assert np.max(np.abs(g - w)) <= 1e-3 * float(np.ptp(w))
    f.close()


@pytest.mark.parametrize("kv_bits", [32, 16])
def test_branches_reference_model(hip, oracle, tiny_stablelm, kv_bits):
    """The reference's tiny StableLM (head width 8): five branches of the
    "Hello abc" prompt, six lockstep tokens each."""
    config, tensors = tiny_stablelm
    branch_case(hip, oracle, config, tensors, HELLO_ABC, 4, [[264], [285], [199], [5], [300]], 6, kv_bits, False)


@pytest.mark.parametrize("prefix,count,kv_bits", [(2, 4, 32), (0, 3, 16), (4, 33, 32)])
def test_branches_prefix_and_count(hip, oracle, tiny_stablelm, prefix, count, kv_bits):
    """A prefix shorter than the resident tokens (the model's tokens past it
    are not seen), prefix 0 (suffix only), and 33 branches (more rows than
    the row-streaming products take: the vector-unit GEMM path)."""
    config, tensors = tiny_stablelm
    config = dict(config, max_position_embeddings=384)
    seeds = [[int(t)] for t in np.random.default_rng(count).integers(0, config["vocab_size"], count)]
    branch_case(hip, oracle, config, tensors, HELLO_ABC + [17, 18], prefix, seeds, 4, kv_bits, False)


@pytest.mark.parametrize("kv_bits", [32, 16])
def test_branches_ragged_suffixes_reference_model(hip, oracle, tiny_stablelm, kv_bits):
    """Private suffixes of lengths 1-9 appended in one call (rows of
    several branches in one chunk, causal within each branch), then four
    lockstep tokens at ragged positions; the suffix caches grow past their
    first capacity (16 positions) on the way."""
    config, tensors = tiny_stablelm
    config = dict(config, max_position_embeddings=384)
    rng = np.random.default_rng(3)
    suffixes = [list(rng.integers(0, 342, n)) for n in (1, 9, 4, 7, 2, 15)]
    branch_case(hip, oracle, config, tensors, HELLO_ABC, 4, suffixes, 4, kv_bits, True)


@pytest.mark.parametrize("mlp,attn,kv_bits", [(W.Q4_K, W.Q6_K, 16), (W.Q4_K, W.Q4_K, 16), (W.Q8_0, W.Q8_0, 32)])
def test_branches_3b_shapes(hip, oracle, mlp, attn, kv_bits):
    """StableLM-3B layer shapes, two layers: the K-quant workload's formats
    (Q6_K attention and classifier, Q4_K MLP), a single-format Q4_K layer
    (row-streamed products on column views of the output-side matrix), and
    Q8_0 with fp32 KV. Five branches with ragged private suffixes (1-70
    tokens: the matrix-core attention reads the shared prefix from the
    model cache and the suffix from the branch cache) on a 70-token prefix,
    then three lockstep tokens."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=512))
    tensors = W.synthetic_stablelm(config, mlp, seed=31, attn_dtype=attn, head_dtype=attn)
    rng = np.random.default_rng(37)
    prompt = list(rng.integers(0, 65536, 70))
    suffixes = [list(rng.integers(0, 65536, n)) for n in (1, 70, 13, 64, 65)]
    oracle.set_threads(8)
    branch_case(hip, oracle, config, tensors, prompt, 70, suffixes, 3, kv_bits, True)


@pytest.mark.parametrize("mlp,attn,kv_bits", [(W.Q4_K, W.Q6_K, 16), (W.Q8_0, W.Q8_0, 32)])
def test_branch_steps_from_graphs_match_direct_launches(hip, mlp, attn, kv_bits):
    """Lockstep branch steps replay a captured graph per attention shape;
    a second session on the same weights and prefix runs with the profiler
    on (every kernel launched directly). Ragged suffixes, then 40 lockstep
    steps (the suffix attention changes shape on the way, so several graphs
    are captured and each is replayed many times, with the host's own work
    and a synchronisation between replays): every step's logits are
    bit-identical, and the caches' growth past 64 positions (which drops
    the graphs) happens within the run. The graph run takes its logits into
    a caller's array (forward's `out`), which must have the rows' shape."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=512))
    tensors = W.synthetic_stablelm(config, mlp, seed=71, attn_dtype=attn, head_dtype=attn)
    rng = np.random.default_rng(73)
    prompt = list(rng.integers(0, 65536, 96))
    suffixes = [list(rng.integers(0, 65536, n)) for n in (1, 30, 7, 24, 12, 3)]
    runs = []
    for direct in (False, True):
        f = hip.StableLMForwarder(config, tensors)
        f.set_kv_bits(kv_bits)
        f.forward(0, prompt, want_logits=False)
        if direct:
            f.profile(True)
        br = f.new_branches(96, len(suffixes))
        rows = [br.append(suffixes)]
        out = np.empty_like(rows[0])  # the graph run also takes the logits into a caller's array
        for s in range(40):
            toks = np.argmax(rows[-1], axis=1).astype(np.int32)
            if direct:
                rows.append(br.forward(toks))
            else:
                assert br.forward(toks, out=out) is out
                rows.append(out.copy())
        with pytest.raises(ValueError):
            br.forward(toks, out=np.empty((2, 3), np.float32))
        br.close()
        f.close()
        runs.append(rows)
    for s, (a, b) in enumerate(zip(*runs)):
        assert np.array_equal(a, b), s


@pytest.mark.parametrize("mlp,attn,count", [(W.Q4_K, W.Q6_K, 6), (W.Q6_K, W.Q4_K, 6), (W.Q4_K, W.Q6_K, 18)])
def test_paired_in_products_match_separate_launches(hip, mlp, attn, count):
    """A branch step's two few-row in-products (q/k/v and gate/up, each in
    its own K-quant format) run as one launch by default (launch stage
    "kq_pair"); with the switch off they run as two launches. Both orders
    of the two formats, 6 branches (one 16-row tile) and 18 (two): the
    ragged appends' and 12 lockstep steps' logits are bit-identical."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=512))
    tensors = W.synthetic_stablelm(config, mlp, seed=83, attn_dtype=attn, head_dtype=attn)
    rng = np.random.default_rng(89)
    prompt = list(rng.integers(0, 65536, 40))
    suffixes = [list(rng.integers(0, 65536, 1 + (7 * i) % 11)) for i in range(count)]
    runs = []
    for paired in (True, False):
        f = hip.StableLMForwarder(config, tensors)
        f.set_kv_bits(16)
        if not paired:
            f.set_launch("kq_pair", 0, 0)
        f.forward(0, prompt, want_logits=False)
        br = f.new_branches(40, count)
        rows = [br.append(suffixes)]
        for s in range(12):
            rows.append(br.forward(np.argmax(rows[-1], axis=1).astype(np.int32)))
        br.close()
        f.close()
        runs.append(rows)
    for s, (a, b) in enumerate(zip(*runs)):
        assert np.all(np.isfinite(a)), s
        assert np.array_equal(a, b), s
