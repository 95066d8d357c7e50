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
