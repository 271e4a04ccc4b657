"""pk_window_split: how pk_decode cuts windows that one launch of the decode
loop cannot take (host arithmetic; runs without a GPU).

One launch takes at most 2^18 - 1 lockstep iterations (the argmax keys' 18-bit
stamp; a window of T frames may take T * (max_symbols + 1) + 4) and at most
(2^31 - 1) / (4 J) frames of enc_proj rows.  The reference's loop has no length
limit (src/parakeet_tdt.cpp:917-967), so longer windows are decoded in pieces
with the state carried.  These tests check the properties the split must have
for that to be exact: the pieces cover each window, every launch stays inside
both bounds, and every piece is longer than the largest duration carry."""
import numpy as np
import pytest

STAMP = (1 << 18) - 1


def pieces(T, k):
    """Piece lengths of a window of T frames in k launches (the documented rule)."""
    return [T // k + (1 if j < T % k else 0) for j in range(k)] if k else []


def check_split(T, max_symbols, J, max_dur):
    from parakeet_amd import pk
    W, k = pk.window_split(T, max_symbols, J, max_dur)
    T = np.asarray(T, np.int64)
    S = max(max_symbols, 1)
    per = [pieces(int(t), int(kk)) for t, kk in zip(T, k)]
    for t, p in zip(T, per):
        assert sum(p) == t                                  # the pieces cover the window
        assert not p or max(p) - min(p) <= 1                # nearly equal
        assert all(x <= W for x in p)
        if len(p) > 1:
            assert min(p) > max_dur - 1                     # longer than any carry_frames
    for j in range(int(k.max()) if len(k) else 0):
        launch = [p[j] for p in per if len(p) > j]
        assert max(launch) * (S + 1) + 4 < STAMP            # iterations of one launch
        assert sum(launch) * J * 4 < (1 << 31)              # enc_proj rows of one launch
    return W, k


def test_no_split_when_one_launch_fits(pkg):
    W, k = check_split([125, 0, 750], 10, 640, 5)
    assert W == 750 and k.tolist() == [1, 0, 1]


def test_stamp_boundary(pkg):
    # the longest window one launch takes at max_symbols S: T * (S + 1) + 4 <= 2^18 - 2
    for S in (1, 5, 10, 100):
        edge = (STAMP - 1 - 4) // (S + 1)
        W, k = check_split([edge], S, 640, 5)
        assert k.tolist() == [1] and W == edge
        W, k = check_split([edge + 1], S, 640, 5)
        assert k[0] >= 2


def test_long_window_b1(pkg):
    # 30,000 frames (40 min of audio at 80 ms) at the default symbol cap
    W, k = check_split([30000], 10, 640, 5)
    assert k[0] >= 2


def test_rows_bound_splits_large_batches(pkg):
    # 512 windows of 2,000 frames: 1.02 M rows exceed the 838,860 rows one launch
    # addresses at J = 640, although every window alone fits the stamp
    T = [2000] * 512
    W, k = check_split(T, 10, 640, 5)
    assert k.min() == 2


def test_ragged_and_empty(pkg):
    rng = np.random.default_rng(5)
    for S in (3, 10, 100):
        T = rng.integers(0, 40000, size=64).tolist() + [0, 1]
        check_split(T, S, 640, 5)


def test_carry_bound_refuses(pkg):
    from parakeet_amd import pk
    # a duration table reaching 10,000 frames: no piece length is longer than its carry
    with pytest.raises(pk.PkError) as e:
        pk.window_split([100000], 10, 640, 10000)
    assert e.value.rc == 5
    W, k = check_split([100000], 10, 640, 4)
    assert k.max() > 1


def test_empty_windows(pkg):
    W, k = check_split([0, 0], 10, 640, 5)
    assert W == 0 and k.tolist() == [0, 0]
    W, k = check_split([], 10, 640, 5)
    assert W == 0
