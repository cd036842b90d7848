"""Pins of the oracle's superblocks (BlockGibbsSpec::new,
crates/thrml-samplers/src/program.rs:28-64; sample_blocks,
crates/thrml-samplers/src/sampling.rs:28-63) that do not retype its sweep.

  - explicit one-block-per-superblock offsets reproduce the default program
    bit for bit (ising.rs:348-349 builds exactly that);
  - grouping blocks with no edge between them changes nothing (no block of
    such a superblock reads another), while grouping adjacent blocks does;
  - one superblock over every free block is a synchronous update: each new
    spin is (u <= sigmoid(2 gamma)) with gamma from the state before the
    sweep (orc_ising_gamma, pinned by the energy-difference identity) and u
    from block b's key sweep_key.split(n_free)[b]; the categorical analogue
    takes the argmax of theta(state before) + Gumbel noise;
  - offsets that are not a partition of the free blocks are rejected.
A planted mistake (a superblock writing each block in place, or keying the
blocks by superblock instead of by flat index) fails the synchronous check.
"""
import numpy as np
import pytest

import pyoracle as orc


def _ising_graph(n, m, seed):
    rng = np.random.default_rng(seed)
    e = set()
    while len(e) < m:
        a, b = rng.integers(0, n, 2)
        if a != b:
            e.add((int(min(a, b)), int(max(a, b))))
    edges = np.array(sorted(e), dtype=np.uint32)
    return edges, rng.normal(0, 0.4, n).astype(np.float32), rng.normal(0, 0.6, len(e)).astype(np.float32)


def _greedy_blocks(n, edges):
    col, _ = orc.greedy_coloring(n, edges)
    return [np.nonzero(col == c)[0].astype(np.uint32) for c in range(int(col.max()) + 1)]


def _start(C, n_total, seed):
    return np.random.default_rng(seed).integers(0, 2, (C, n_total)).astype(np.uint8)


def test_explicit_trivial_offsets_equal_default():
    n = 60
    edges, b, w = _ising_graph(n, 150, 3)
    blocks = _greedy_blocks(n, edges)
    nb = len(blocks)
    p0 = orc.Ising(n, edges, b, w, 0.9, blocks)
    p1 = orc.Ising(n, edges, b, w, 0.9, blocks, superblocks=list(range(nb + 1)))
    st = _start(5, p0.n_total, 4)
    a, _ = p0.run_blocks(77, st, 4)
    c, _ = p1.run_blocks(77, st, 4)
    np.testing.assert_array_equal(a, c)


def test_grouping_non_adjacent_blocks_is_sequential():
    # two disjoint graphs: blocks of graph 1 never read blocks of graph 2
    n1 = 30
    e1, b1, w1 = _ising_graph(n1, 60, 5)
    e2, b2, w2 = _ising_graph(n1, 60, 6)
    edges = np.concatenate([e1, e2 + n1])
    b = np.concatenate([b1, b2])
    w = np.concatenate([w1, w2])
    g1 = _greedy_blocks(n1, e1)
    g2 = [x + n1 for x in _greedy_blocks(n1, e2)]
    k = min(len(g1), len(g2))
    # free blocks: g1[0], g2[0], g1[1], g2[1], ...; superblocks pair them up
    blocks, off = [], [0]
    for i in range(k):
        blocks += [g1[i], g2[i]]
        off.append(len(blocks))
    for extra in g1[k:] + g2[k:]:
        blocks.append(extra)
        off.append(len(blocks))
    seq = orc.Ising(2 * n1, edges, b, w, 1.1, blocks)
    grp = orc.Ising(2 * n1, edges, b, w, 1.1, blocks, superblocks=off)
    st = _start(4, seq.n_total, 7)
    a, _ = seq.run_blocks(91, st, 3)
    c, _ = grp.run_blocks(91, st, 3)
    np.testing.assert_array_equal(a, c)


def test_grouping_adjacent_blocks_changes_the_sweep():
    n = 64
    edges, b, w = _ising_graph(n, 200, 8)
    blocks = _greedy_blocks(n, edges)
    seq = orc.Ising(n, edges, b, w, 1.3, blocks)
    grp = orc.Ising(n, edges, b, w, 1.3, blocks, superblocks=[0, len(blocks)])
    st = _start(8, seq.n_total, 9)
    a, _ = seq.run_blocks(5, st, 2)
    c, _ = grp.run_blocks(5, st, 2)
    assert (a != c).any()


def _sweep_block_keys(key, C, n_free):
    """Per chain: block keys of the single sweep of run_blocks(n_iters = 1)."""
    out = []
    for ck in orc.rng_split(key, C):
        sk = orc.rng_split(ck, 1)[0]
        out.append(orc.rng_split(sk, n_free))
    return out


def test_one_superblock_is_a_synchronous_ising_update():
    n = 50
    edges, b, w = _ising_graph(n, 140, 10)
    blocks = _greedy_blocks(n, edges)
    # one superblock over the free blocks; the last block stays clamped
    free, clamped = blocks[:-1], blocks[-1:]
    nf = len(free)
    beta = 0.8
    p = orc.Ising(n, edges, b, w, beta, free, clamped, superblocks=[0, nf])
    C, key = 3, 2024
    st = _start(C, p.n_total, 11)
    got, _ = p.run_blocks(key, st, 1)
    keys = _sweep_block_keys(key, C, nf)
    lens = [x.size for x in free]
    for c in range(C):
        gam = p.gamma(st[c])  # gamma of every free position from the state before
        exp = st[c].copy()
        pos = 0
        for blk in range(nf):
            k8 = orc.seed_from_u64(keys[c][blk])
            for i in range(lens[blk]):
                u = np.float32((orc.stream_word(k8, i) >> 8) * 2.0**-24)
                prob = orc.sigmoid(np.float32(2.0) * gam[pos + i])
                exp[pos + i] = 1 if u <= prob else 0
            pos += lens[blk]
        np.testing.assert_array_equal(got[c], exp)


def test_one_superblock_is_a_synchronous_categorical_update():
    rng = np.random.default_rng(12)
    n, q = 36, 5
    edges, _, _ = _ising_graph(n, 90, 12)
    W = rng.normal(0, 0.5, (edges.shape[0], q, q)).astype(np.float32)
    bias = rng.normal(0, 0.5, (n, q)).astype(np.float32)
    blocks = _greedy_blocks(n, edges)
    nf = len(blocks)
    p = orc.Potts(n, q, edges, W, bias, blocks, superblocks=[0, nf])
    C, key = 4, 404
    st = rng.integers(0, q, (C, p.n_total)).astype(np.uint8)
    got, _ = p.run_blocks(key, st, 1)
    keys = _sweep_block_keys(key, C, nf)
    for c in range(C):
        theta = p.theta(st[c])
        exp = st[c].copy()
        pos = 0
        for blk in range(nf):
            k8 = orc.seed_from_u64(keys[c][blk])
            for i in range(blocks[blk].size):
                v = [theta[pos + i][j] + orc.gumbel(orc.stream_word(k8, i * q + j)) for j in range(q)]
                exp[pos + i] = int(np.argmax(np.asarray(v, np.float32)))
            pos += blocks[blk].size
        np.testing.assert_array_equal(got[c], exp)


def test_mixed_superblocks_match_a_composition_of_runs():
    """[A, B] grouped, then C alone: C reads A and B's new states.  Checked by
    splitting the sweep: the grouped part is the synchronous update above,
    the last block a one-block update with the next key."""
    n = 40
    edges, b, w = _ising_graph(n, 110, 13)
    blocks = _greedy_blocks(n, edges)
    assert len(blocks) >= 3
    nf = len(blocks)
    p = orc.Ising(n, edges, b, w, 1.0, blocks, superblocks=[0, 2] + list(range(3, nf + 1)))
    C, key = 2, 555
    st = _start(C, p.n_total, 14)
    got, _ = p.run_blocks(key, st, 1)
    keys = _sweep_block_keys(key, C, nf)
    lens = [x.size for x in blocks]
    offs = np.concatenate([[0], np.cumsum(lens)])
    for c in range(C):
        cur = st[c].copy()
        # superblock 0: blocks 0 and 1 from the state before
        gam = p.gamma(cur)
        new = cur.copy()
        for blk in (0, 1):
            k8 = orc.seed_from_u64(keys[c][blk])
            for i in range(lens[blk]):
                u = np.float32((orc.stream_word(k8, i) >> 8) * 2.0**-24)
                new[offs[blk] + i] = 1 if u <= orc.sigmoid(np.float32(2.0) * gam[offs[blk] + i]) else 0
        cur = new
        # later superblocks one block each, in order
        for blk in range(2, nf):
            gam = p.gamma(cur)
            k8 = orc.seed_from_u64(keys[c][blk])
            for i in range(lens[blk]):
                u = np.float32((orc.stream_word(k8, i) >> 8) * 2.0**-24)
                cur[offs[blk] + i] = 1 if u <= orc.sigmoid(np.float32(2.0) * gam[offs[blk] + i]) else 0
        np.testing.assert_array_equal(got[c], cur)


@pytest.mark.parametrize("off,msg", [
    ([1, 3], "start at 0"),
    ([0, 2], "end at the number"),
    ([0, 2, 1, 3], "must not decrease"),
])
def test_invalid_offsets_rejected(off, msg):
    n = 12
    edges, b, w = _ising_graph(n, 20, 15)
    blocks = [np.arange(0, 4, dtype=np.uint32), np.arange(4, 8, dtype=np.uint32),
              np.arange(8, 12, dtype=np.uint32)]
    with pytest.raises(ValueError, match=msg):
        orc.Ising(n, edges, b, w, 1.0, blocks, superblocks=off)


def test_empty_superblock_is_a_no_op():
    n = 30
    edges, b, w = _ising_graph(n, 50, 16)
    blocks = _greedy_blocks(n, edges)
    nb = len(blocks)
    p0 = orc.Ising(n, edges, b, w, 1.0, blocks)
    p1 = orc.Ising(n, edges, b, w, 1.0, blocks, superblocks=[0, 0] + list(range(1, nb + 1)))
    st = _start(3, p0.n_total, 17)
    np.testing.assert_array_equal(p0.run_blocks(8, st, 3)[0], p1.run_blocks(8, st, 3)[0])


def test_opbyop_follows_superblocks():
    n = 40
    edges, b, w = _ising_graph(n, 100, 18)
    blocks = _greedy_blocks(n, edges)
    nf = len(blocks)
    p = orc.Ising(n, edges, b, w, 0.7, blocks, superblocks=[0, 2] + list(range(3, nf + 1)))
    st = _start(3, p.n_total, 19)
    np.testing.assert_array_equal(p.run_blocks(31, st, 3)[0], p.run_blocks_opbyop(31, st, 3))
