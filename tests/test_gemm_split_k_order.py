"""The split-K prefill GEMM's combine order is fixed_tree's (CPU only).

q4k_gemm_sk_kernel cuts a row's R super-blocks into chunks: the balanced
trees of R's binary digits, from the highest, each cut into pieces of C
leaves (a tree smaller than C is one piece); each wave folds one chunk, and
wave 0 adds the chunk values pairwise inside each tree and folds the trees
right to left.  This restates that order symbolically and checks that it
builds exactly the tree of fixed_tree (src/ops/quant.rs:461-476: level by
level, pairs (2t, 2t+1), an odd last block passed up) over R leaves, for
every row length the kernel takes and every piece size it may pick; a wrong
digit order, a left fold or a mis-sized piece changes the tree.  The GPU
parity tests check the kernel's results against the oracle.
"""
import pytest

MAX_WAVES = 12  # kSkMaxWaves


def fixed_tree(leaves):
    p = list(leaves)
    while len(p) > 1:
        p = [(p[2 * t], p[2 * t + 1]) if 2 * t + 1 < len(p) else p[2 * t] for t in range((len(p) + 1) // 2)]
    return p[0]


def pieces(R, C, k):
    return (1 << k) // C if (1 << k) >= C else 1


def chunks(R, C):
    return sum(pieces(R, C, k) for k in range(6, -1, -1) if (R >> k) & 1)


def split_k_tree(R, C):
    # the waves' chunks, in wave order
    vals, base = [], 0
    for k in range(6, -1, -1):
        if not (R >> k) & 1:
            continue
        size = 1 << k
        n, sz = (size // C, C) if size >= C else (1, size)
        vals += [fixed_tree(range(base + i * sz, base + (i + 1) * sz)) for i in range(n)]
        base += size
    assert base == R and len(vals) == chunks(R, C)
    # wave 0: the trees from the lowest digit up, each reduced pairwise
    acc = None
    for k in range(7):
        if not (R >> k) & 1:
            continue
        c0 = sum(pieces(R, C, k2) for k2 in range(k + 1, 7) if (R >> k2) & 1)
        v = vals[c0:c0 + pieces(R, C, k)]
        st = 1
        while st < len(v):
            for i in range(0, len(v) - st, 2 * st):
                v[i] = (v[i], v[i + st])
            st *= 2
        acc = v[0] if acc is None else (v[0], acc)
    return acc


@pytest.mark.parametrize("R", range(1, 128))
def test_split_k_combine_is_fixed_tree(R):
    valid = [C for C in (1, 2, 4, 8, 16) if chunks(R, C) <= MAX_WAVES]
    assert valid, "every row length below 128 super-blocks has a piece size"
    for C in valid:
        assert split_k_tree(R, C) == fixed_tree(range(R)), (R, C)


def test_a_serial_fold_of_the_chunks_would_differ():
    # adding the chunk values in wave order (a left fold) is a different
    # tree: with R = 7 and single-leaf pieces, ((0+1)+2)+... against
    # ((0+1)+(2+3)) + ((4+5)+6)
    R, C = 7, 1
    left = None
    for v in range(R):
        left = v if left is None else (left, v)
    assert split_k_tree(R, C) == fixed_tree(range(R)) != left
