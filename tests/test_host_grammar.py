"""The host walk that builds the verify rows' grammar masks (gravityocr_amd.sampling.grammar_masks, after
fulldraft_bitmask, selfspec_sampling.py:305-337), against brute force on a position-dependent grammar: row j of a
sequence allows exactly what the grammar allows after [a0, d_1..d_j]; rows past a draft token its previous row forbids
stay all-allowed; sequences without a grammar are all-allowed; every grammar leaves in the state it came in."""
import numpy as np

from tests.helpers import PositionGrammar


def _unpack(mask_row, V):
    w = np.asarray(mask_row, dtype=np.int32).view(np.uint32).astype(np.uint64)
    return [bool((int(w[t >> 5]) >> (t & 31)) & 1) for t in range(V)]


def test_grammar_masks_follow_the_walk():
    from gravityocr_amd.sampling import grammar_masks
    V, K = 70, 5
    rng = np.random.default_rng(0)
    g0 = PositionGrammar(V, [4, 8])
    g2 = PositionGrammar(V, [1])
    cand = [[int(x) for x in rng.integers(0, V, K)] for _ in range(3)]
    # make sequence 0's window allowed throughout, sequence 2's forbidden at d_2
    ref = PositionGrammar(V, g0.acc)
    cand[0][0] = next(t for t in range(V) if ref.allowed(t)); ref.acc.append(cand[0][0])
    for j in range(1, K):
        cand[0][j] = next(t for t in range(V) if ref.allowed(t) and t > 10 * j % V); ref.acc.append(cand[0][j])
    ref2 = PositionGrammar(V, g2.acc)
    cand[2][0] = next(t for t in range(V) if ref2.allowed(t)); ref2.acc.append(cand[2][0])
    cand[2][1] = next(t for t in range(V) if ref2.allowed(t)); ref2.acc.append(cand[2][1])
    cand[2][2] = next(t for t in range(V) if not ref2.allowed(t))
    before0, before2 = list(g0.acc), list(g2.acc)
    m = grammar_masks([g0, None, g2], cand, V).numpy()
    assert g0.acc == before0 and g2.acc == before2
    for b, g, n_rows in ((0, before0, K), (2, before2, 2)):
        for j in range(K):
            got = _unpack(m[b * K + j], V)
            if j < n_rows:
                st = PositionGrammar(V, g + cand[b][:j + 1])
                assert got == [st.allowed(t) for t in range(V)], (b, j)
            else:
                assert all(got), (b, j)                    # past the forbidden d_2: all-allowed
    for j in range(K):
        assert all(_unpack(m[K + j], V))                   # no grammar


def test_grammar_masks_current_state_row():
    """first_accepted=False: row 0 is the grammar's current state (the a0 row and the AR step)."""
    from gravityocr_amd.sampling import grammar_masks
    V = 40
    g = PositionGrammar(V, [3, 5, 7])
    m = grammar_masks([g], [[0]], V, first_accepted=False).numpy()
    assert _unpack(m[0], V) == [g.allowed(t) for t in range(V)] and g.acc == [3, 5, 7]
