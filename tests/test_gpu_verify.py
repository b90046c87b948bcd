"""Token side of a speculative verify round on the device
(`dbi_spec_verify_async`, `dbi_kv_verify_commit`): the argmax of each of the
k+1 logit rows (sample.cpp:11-28) and the merge against the draft
(speculative.cpp:10-23), bit-exact with the oracle (`ok_argmax`,
`ok_spec_merge`), which is pinned by the reference's own vectors.

Covered: the golden argmax vectors of tests/sample_test.cpp:38-50 and merge
vectors of tests/speculative_test.cpp:104-133; NaN (slot 0 and later),
signed zeros and infinities; rows of heavy ties; vocab sizes from 1 to 262144
(one to 64 workgroups per row) and k from 1 to 64; back-to-back calls (the
arrival counter resets itself); the commit's truncation and its error paths;
graph replay with new logits between replays.
"""
import json
import os

import numpy as np
import pytest

import pyoracle
from dbinfer_amd.kv import F32, DbiError, HipKV
from helpers import GOLDEN, normal

pytestmark = pytest.mark.gpu

NAN, INF = np.float32("nan"), np.float32("inf")


@pytest.fixture(scope="module")
def torch():
    return pytest.importorskip("torch")


@pytest.fixture(scope="module")
def kv():
    h = HipKV(1, 64, 1, 64)
    yield h
    h.close()


def run(torch, kv, logits, draft):
    """verified argmaxes and accepted count from the device."""
    logits = np.ascontiguousarray(logits, np.float32)
    rows, vocab = logits.shape
    assert len(draft) == rows - 1
    lt = torch.from_numpy(logits).cuda()
    dt = torch.tensor(np.asarray(draft, np.int32), device="cuda")
    ver = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
    acc = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    kv.set_stream(torch.cuda.current_stream().cuda_stream)
    kv.spec_verify_async(rows - 1, vocab, lt.data_ptr(), dt.data_ptr(), ver.data_ptr(),
                         acc.data_ptr())
    torch.cuda.synchronize()
    return ver.cpu().numpy().tolist(), int(acc.item())


def expect(logits, draft):
    ver = [pyoracle.argmax(r) for r in np.asarray(logits, np.float32)]
    acc, merged = pyoracle.spec_merge(draft, ver)
    assert merged == ver[: acc + 1]
    return ver, acc


ARGMAX = json.load(open(os.path.join(GOLDEN, "argmax_cases.json")))["cases"]
MERGE = json.load(open(os.path.join(GOLDEN, "spec_merge_cases.json")))["cases"]


@pytest.mark.parametrize("case", ARGMAX)
def test_golden_argmax(torch, kv, case):
    row = np.asarray(case["logits"], np.float32)
    ver, _ = run(torch, kv, np.stack([row, row]), [0])
    assert ver == [case["index"]] * 2


@pytest.mark.parametrize("case", MERGE)
def test_golden_merge(torch, kv, case):
    vocab = 128
    tgt = case["target"]
    logits = np.full((len(tgt), vocab), -1.0, np.float32)
    for i, t in enumerate(tgt):
        logits[i, t] = 2.0
    ver, acc = run(torch, kv, logits, case["draft"])
    assert ver == tgt
    assert acc == case["accepted"] and ver[: acc + 1] == case["out"]


SPECIAL = [
    [NAN, 1.0, 2.0], [1.0, NAN, 2.0], [NAN, NAN, NAN], [-0.0, 0.0, -0.0], [0.0, -0.0, 0.0],
    [-INF, -INF, -INF], [-INF, NAN, -1.0], [3.0, INF, INF], [-1.0, -INF, -0.5],
]


@pytest.mark.parametrize("row", SPECIAL)
def test_special_values(torch, kv, row):
    r = np.asarray(row, np.float32)
    want = pyoracle.argmax(r)
    ver, _ = run(torch, kv, np.stack([r, r]), [want])
    assert ver == [want, want]


@pytest.mark.parametrize("vocab", [1, 7, 1000, 4096, 4097, 32000, 151936, 262144])
@pytest.mark.parametrize("k", [1, 4, 8])
def test_random_rows(torch, kv, vocab, k):
    rng = np.random.default_rng(vocab * 131 + k)
    rows = k + 1
    logits = rng.integers(-3, 4, (rows, vocab)).astype(np.float32)  # heavy ties
    logits[1::2] = normal(vocab + k, (rows - 1) // 2 + 1, vocab)[: logits[1::2].shape[0]]
    nan = rng.random((rows, vocab)) < 0.05
    logits[nan] = NAN
    if rows > 2:
        logits[2, 0] = NAN  # slot-0 NaN: answer 0
    if vocab > 5:
        j = rng.integers(1, vocab)
        logits[0, j] = INF  # a single +inf wins
        logits[-1, :] = -0.0
        logits[-1, vocab - 1] = 0.0  # equal to -0.0: answer 0
    want = [pyoracle.argmax(r) for r in logits]
    # draft agrees with a prefix of the argmaxes, then diverges
    cut = int(rng.integers(0, k + 1))
    draft = [want[i] if i < cut else want[i] + 1 for i in range(k)]
    ver, acc = run(torch, kv, logits, draft)
    assert ver == want
    assert (acc, ver[: acc + 1]) == pyoracle.spec_merge(draft, want)
    assert acc == cut


def test_max_draft_and_back_to_back(torch, kv):
    """k = 64 (65 rows), then smaller calls on the same handle: the arrival
    counter the last workgroup resets serves every call."""
    for it, (k, vocab) in enumerate([(64, 50000), (3, 151936), (64, 333), (1, 1)]):
        logits = normal(900 + it, k + 1, vocab)
        want, _ = expect(logits, [0] * k)
        draft = list(want[:k])
        if it % 2:
            draft[k // 2] = -1
        ver, acc = run(torch, kv, logits, draft)
        assert ver == want
        assert acc == (k if it % 2 == 0 else k // 2)


def test_verify_commit_truncates(torch):
    L, cap, nkv, hd = 2, 64, 2, 64
    kv = HipKV(L, cap, nkv, hd)
    pos, k, vocab = 20, 5, 3000
    P = nkv * hd
    K, V = normal(1, L, pos + k + 1, P), normal(2, L, pos + k + 1, P)
    for l in range(L):
        kv.append_n(l, 0, K[l], V[l])
    assert kv.n_seen == pos + k + 1
    logits = normal(3, k + 1, vocab)
    want = [pyoracle.argmax(r) for r in logits]
    draft = want[:2] + [want[2] + 1] + want[3:k]
    lt = torch.from_numpy(logits).cuda()
    kv.set_stream(torch.cuda.current_stream().cuda_stream)
    acc, merged = kv.verify_commit(pos, k, vocab, lt.data_ptr(), draft)
    assert (acc, merged) == pyoracle.spec_merge(draft, want) == (2, want[:3])
    assert kv.n_seen == pos + acc + 1
    # a fully accepted round keeps every row and emits the bonus token
    for l in range(L):
        kv.append_n(l, pos + acc + 1, K[l, : k + 1], V[l, : k + 1])
    p2 = pos + acc + 1
    acc2, merged2 = kv.verify_commit(p2, k, vocab, lt.data_ptr(), want[:k])
    assert (acc2, merged2) == (k, want)
    assert kv.n_seen == p2 + k + 1
    kv.close()


def test_verify_errors(torch, kv):
    lt = torch.zeros(66, 8, device="cuda")
    it = torch.zeros(66, dtype=torch.int32, device="cuda")
    for k, vocab, msg in [(0, 8, "1 <= k <= 64"), (65, 8, "1 <= k <= 64"),
                          (2, 0, "vocab"), (2, (1 << 30) + 1, "vocab")]:
        with pytest.raises(DbiError) as e:
            kv.spec_verify_async(k, vocab, lt.data_ptr(), it.data_ptr(), it.data_ptr(),
                                 it.data_ptr())
        assert msg in e.value.message
    with pytest.raises(DbiError) as e:
        kv.spec_verify_async(2, 8, 0, it.data_ptr(), it.data_ptr(), it.data_ptr())
    assert "null" in e.value.message
    h = HipKV(1, 32, 1, 64)
    h.append_n(0, 0, normal(4, 10, 64), normal(5, 10, 64))
    with pytest.raises(DbiError) as e:
        h.verify_commit(6, 4, 8, lt.data_ptr(), [0] * 4)  # pos + k + 1 = 11 > 10
    assert "pos + k + 1 <= n_seen" in e.value.message
    assert h.n_seen == 10
    assert h.verify_commit(5, 4, 8, lt.data_ptr(), [0] * 4) == (4, [0] * 5)  # zeros: all 0
    assert h.n_seen == 10
    h.close()


def test_verify_graph_replay(torch):
    """Captured after one eager call; each replay reads the logits written
    since, with eager work and synchronizations between replays."""
    k, vocab = 4, 151936
    kv = HipKV(1, 64, 1, 64)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        lt = torch.zeros(k + 1, vocab, device="cuda")
        dt = torch.zeros(k, dtype=torch.int32, device="cuda")
        ver = torch.zeros(k + 1, dtype=torch.int32, device="cuda")
        acc = torch.zeros(1, dtype=torch.int32, device="cuda")
        kv.set_stream(s.cuda_stream)
        kv.spec_verify_async(k, vocab, lt.data_ptr(), dt.data_ptr(), ver.data_ptr(),
                             acc.data_ptr())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        kv.spec_verify_async(k, vocab, lt.data_ptr(), dt.data_ptr(), ver.data_ptr(),
                             acc.data_ptr())
    torch.cuda.synchronize()
    for rep in range(5):
        logits = normal(70 + rep, k + 1, vocab)
        want = [pyoracle.argmax(r) for r in logits]
        draft = want[:k]
        if rep % 2:
            draft[rep % k] = -3
        lt.copy_(torch.from_numpy(logits))
        dt.copy_(torch.tensor(draft, dtype=torch.int32))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert ver.cpu().numpy().tolist() == want, f"replay {rep}"
        assert int(acc.item()) == pyoracle.spec_merge(draft, want)[0], f"replay {rep}"
        _ = (lt * 2).sum()  # eager work between replays
    kv.close()
