"""The depth ladder (crates/model/src/ladder.rs) — host code, no device needed:
known answers worked by hand from the rule (first and last layer, then the
midpoint of the widest gap, the leftmost of equal gaps) and its invariants."""
import rustyneedle_amd as rn


def test_known_orders():
    assert rn.ladder_order(0) == [] and rn.ladder_order(1) == [0]
    assert rn.ladder_order(2) == [0, 1]
    assert rn.ladder_order(5) == [0, 4, 2, 1, 3]
    assert rn.ladder_order(8) == [0, 7, 3, 5, 1, 2, 4, 6]  # (3, 7) is wider than (0, 3)


def test_orders_are_permutations_with_the_widest_gap_rule():
    for layers in range(2, 40):
        order = rn.ladder_order(layers)
        assert sorted(order) == list(range(layers))
        chosen = sorted(order[:2])
        for nxt in order[2:]:
            gaps = [(b - a, -a, a, b) for a, b in zip(chosen, chosen[1:]) if b - a > 1]
            _, _, a, b = max(gaps)
            assert nxt == (a + b) // 2
            chosen = sorted(chosen + [nxt])


def test_select():
    assert rn.ladder_select(8, 3) == [0, 3, 7]
    assert rn.ladder_select(8, 8) == list(range(8))
    assert rn.ladder_select(8, 1) is None and rn.ladder_select(8, 9) is None
    assert rn.ladder_select(1, 1) == [0] and rn.ladder_select(0, 0) == []


def test_reference_known_answers():
    """crates/model/tests/ladder.rs:3-29, the reference's own expected values."""
    assert rn.ladder_order(20) == [0, 19, 9, 14, 4, 6, 11, 16, 2, 7, 12, 17, 1, 3, 5, 8, 10, 13, 15, 18]
    assert rn.ladder_select(20, 2) == [0, 19]
    assert rn.ladder_select(20, 4) == [0, 9, 14, 19]
    assert rn.ladder_select(20, 8) == [0, 4, 6, 9, 11, 14, 16, 19]
    assert rn.ladder_select(20, 12) == [0, 2, 4, 6, 7, 9, 11, 12, 14, 16, 17, 19]
    assert rn.ladder_select(20, 20) == list(range(20))
    assert rn.ladder_select(20, 1) is None and rn.ladder_select(20, 21) is None
    eight, four = rn.ladder_select(8, 8), rn.ladder_select(8, 4)
    assert all(layer in eight for layer in four)
    assert rn.ladder_select(8, 2) == [0, 7]
