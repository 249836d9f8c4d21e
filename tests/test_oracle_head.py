"""Pins the output-head oracle (oracle/ref_head.py).  No GPU."""
import numpy as np
import torch

from oracle import ref_head as H


def test_nucleus_limits():
    torch.manual_seed(0)
    logits = torch.randn(3, 50)
    kept0, p0 = H.nucleus(logits, 1.0, 0.0)
    assert (kept0.sum(-1) == 1).all()
    assert torch.equal(kept0.float().argmax(-1), logits.argmax(-1))
    assert torch.allclose(p0.sum(-1), torch.ones(3))
    kept1, p1 = H.nucleus(logits, 0.7, 1.5)
    assert kept1.all()
    torch.testing.assert_close(p1, torch.softmax(logits / 0.7, -1))


def test_nucleus_hand_example():
    # probabilities 0.5, 0.3, 0.15, 0.05 (in shuffled vocabulary order), top_p 0.75:
    # mass before: 0, 0.5, 0.8 (> 0.75, dropped), 0.95 (dropped) -> keep the top two
    p = torch.tensor([[0.15, 0.5, 0.05, 0.3]])
    kept, q = H.nucleus(torch.log(p), 1.0, 0.75)
    assert kept.tolist() == [[False, True, False, True]]
    torch.testing.assert_close(q, torch.tensor([[0.0, 0.625, 0.0, 0.375]]))


def test_nucleus_ties_in_vocabulary_order():
    # probabilities proportional to 1, e, e, e, 1: p_e = e / (3e + 2), p_1 = 1 / (3e + 2).
    # Sorted with ties in vocabulary order: 1, 2, 3 (mass before 0, p_e, 2 p_e), then 0, 4.
    logits = torch.tensor([[0.0, 1.0, 1.0, 1.0, 0.0]])
    e = float(np.e)
    p_e, p_1 = e / (3 * e + 2), 1 / (3 * e + 2)
    kept, _ = H.nucleus(logits, 1.0, 0.0)
    assert kept.tolist() == [[False, True, False, False, False]]        # only the first maximum
    kept, q = H.nucleus(logits, 1.0, 1.5 * p_e)                          # 2 p_e > 1.5 p_e: token 3 dropped
    assert kept.tolist() == [[False, True, True, False, False]]
    torch.testing.assert_close(q, torch.tensor([[0.0, 0.5, 0.5, 0.0, 0.0]]))
    kept, _ = H.nucleus(logits, 1.0, 3 * p_e + 0.5 * p_1)                # token 0 at 3 p_e, token 4 at 3 p_e + p_1
    assert kept.tolist() == [[True, True, True, True, False]]


def test_nucleus_rule_float64():
    g = torch.Generator().manual_seed(1)
    for top_p, tied in ((0.1, False), (0.5, False), (0.9, False), (0.99, False), (0.5, True), (0.9, True)):
        logits = torch.randn(4, 300, generator=g) * 3
        if tied:
            logits = torch.round(logits * 2) / 2          # many equal probabilities
        kept, _ = H.nucleus(logits, 0.8, top_p)
        pr = torch.softmax(logits.double() / 0.8, -1).numpy()
        for r in range(4):
            order = np.argsort(-pr[r], kind="stable")
            before = np.concatenate([[0.0], np.cumsum(pr[r][order])[:-1]])
            want = np.zeros(300, bool)
            want[order[before <= top_p]] = True
            # fp32 vs fp64 can only disagree where the mass before a token is within rounding of top_p
            diff = np.nonzero(want != kept[r].numpy())[0]
            for i in diff:
                b = before[np.nonzero(order == i)[0][0]]
                assert abs(b - top_p) < 1e-5, (top_p, r, i, b)


def test_greedy_ties_to_first():
    logits = torch.tensor([[1.0, 3.0, 3.0, 2.0], [5.0, 5.0, 5.0, 5.0]])
    assert H.greedy(logits).tolist() == [1, 0]


def test_lm_head_logits_one_hot_and_float64():
    """forward.py:67-72 restated: one-hot vocabulary rows select single normed hidden entries
    exactly; a weight of powers of two scales the logits exactly; random weights agree with a
    float64 product of the same bf16 operands to fp32 summation accuracy."""
    from oracle.ref_ops import rms_norm
    g = torch.Generator().manual_seed(5)
    h = torch.randn(3, 1, 256, generator=g).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn(256, generator=g)).to(torch.bfloat16)
    hn = rms_norm(h, gamma, 1e-6).float().reshape(3, 256)
    sel = torch.tensor([0, 17, 255, 128, 3])
    w = torch.zeros(5, 256, dtype=torch.bfloat16)
    w[torch.arange(5), sel] = 1.0
    got = H.lm_head_logits(h, gamma, w, 1e-6).reshape(3, 5)
    assert torch.equal(got, hn[:, sel])
    w2 = torch.zeros(5, 256, dtype=torch.bfloat16)
    w2[torch.arange(5), sel] = torch.tensor([2.0, -4.0, 0.5, 8.0, -0.25], dtype=torch.bfloat16)
    got2 = H.lm_head_logits(h, gamma, w2, 1e-6).reshape(3, 5)
    assert torch.equal(got2, hn[:, sel] * torch.tensor([2.0, -4.0, 0.5, 8.0, -0.25]))
    wr = (torch.randn(64, 256, generator=g) * 0.05).to(torch.bfloat16)
    got3 = H.lm_head_logits(h, gamma, wr, 1e-6).reshape(3, 64).double()
    want = hn.double() @ wr.double().T
    assert (got3 - want).abs().max() < 1e-5
