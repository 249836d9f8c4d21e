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


def test_nucleus_rule_float64():
    g = torch.Generator().manual_seed(1)
    for top_p in (0.1, 0.5, 0.9, 0.99):
        logits = torch.randn(4, 300, generator=g) * 3
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
