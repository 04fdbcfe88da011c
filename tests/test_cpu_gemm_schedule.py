"""CPU: validation and tile schedule of the grouped Newton-Schulz GEMM launch.

apexw_gemm_grouped_items / apexw_gemm_grouped_schedule are host functions of
the library (no GPU): they check every problem of a grouped launch and assign
its output tiles to the persistent workgroups.  The pointers below are
aligned stand-ins; nothing is dereferenced.
"""

import numpy as np
import pytest

from apexw_amd import _lib

T = _lib.GEMM_TILE
NS_A, NS_B, NS_C = 3.4445, -4.7750, 2.0315


def _prob(a, b, et, c, ct, m, n, k, lda, ldb, lde, ldc, ldct, alpha=1.0, beta=0.0, flags=0):
    return (a, b, et, c, ct, m, n, k, lda, ldb, lde, ldc, ldct, alpha, beta, flags, 0)


def _ns_problems(m, n, batch, base):
    """The three Newton-Schulz products of `batch` m x n work matrices (m <= n),
    as the optimizer issues them (X' = B X + a X with X as [K x N] rows and the
    addend taken from that operand)."""
    xx, aa, bx = [], [], []
    for e in range(batch):
        x, a, b, nx = (base + (4 * e + i) * (1 << 32) for i in range(4))
        xx.append(_prob(x, x, 0, a, a, m, m, n, n, n, 0, m, m, flags=_lib.GEMM_SYM))
        aa.append(_prob(a, a, a, b, b, m, m, m, m, m, m, m, m, NS_C, NS_B, _lib.GEMM_SYM))
        bx.append(_prob(b, x, 0, nx, 0, m, n, m, m, n, 0, n, 0, 1.0, NS_A, _lib.GEMM_B_KN | _lib.GEMM_ADD_B))
    return xx, aa, bx


def _c5_phases():
    """Llama-3-8B layer Muon matrices: q, o (4096^2, batched) and gate/up (+ down) at 4096 x 14336."""
    q = _ns_problems(4096, 4096, 2, 1 << 40)
    gu = _ns_problems(4096, 14336, 2, 2 << 40)
    d = _ns_problems(4096, 14336, 1, 3 << 40)
    return [q[i] + gu[i] + d[i] for i in range(3)]


def _decode(items):
    """(problem, tile row, tile column, part): part 0 = whole tile, 1 / 2 = upper / lower 128-row half."""
    return items >> 24, (items >> 11) & 0x7FF, items & 0x7FF, (items >> 22) & 3


def _expected_tiles(probs):
    out = set()
    for pi, p in enumerate(probs):
        m, n, sym = p[5], p[6], p[15] & _lib.GEMM_SYM
        for tm in range(m // T):
            for tn in range(n // T):
                if not sym or tm <= tn:
                    out.add((pi, tm, tn))
    return out


@pytest.mark.parametrize("phase,kind", [(0, _lib.GEMM_OUT_C | _lib.GEMM_OUT_CT),
                                        (1, _lib.GEMM_OUT_C | _lib.GEMM_OUT_CT | _lib.GEMM_ADD),
                                        (2, _lib.GEMM_OUT_C | _lib.GEMM_ADD | _lib.GEMM_KIND_NN)])
def test_schedule_covers_every_tile_once_in_balanced_bands(phase, kind):
    probs = _c5_phases()[phase]
    items, offsets, n_wg, got_kind = _lib.gemm_schedule(_lib.gemm_problems(probs))
    nq = _lib.GEMM_QUEUES
    assert got_kind == kind and len(offsets) == nq + 1
    assert n_wg == nq * np.diff(offsets).max()          # one workgroup per slot of the longest queue
    assert offsets[0] == 0 and offsets[-1] == len(items) and np.all(np.diff(offsets) >= 0)
    p, tm, tn, part = _decode(items.astype(np.int64))
    assert np.all(part == 0)                            # no CU count given: whole tiles only
    got = list(zip(p.tolist(), tm.tolist(), tn.tolist()))
    assert len(got) == len(set(got)), "a tile is scheduled twice"
    assert set(got) == _expected_tiles(probs)
    # symmetric problems: only tiles on or above the diagonal
    sym = np.array([probs[i][15] & _lib.GEMM_SYM for i in p.tolist()], dtype=bool)
    assert np.all(tm[sym] <= tn[sym])
    # every queue holds an equal share of the cost (K tiles + 2 per epilogue
    # stream: C, Ct, E), within two of the longest tiles
    epi = 2 * bin(kind).count("1")
    ktiles = np.array([probs[i][7] // _lib.GEMM_KTILE for i in p.tolist()])
    loads = np.array([(ktiles[offsets[q]:offsets[q + 1]] + epi).sum() for q in range(nq)])
    assert loads.max() - loads.min() <= 2 * (ktiles.max() + epi), loads
    # per problem, queue q holds the q-th contiguous band of its locality order
    # and every queue gets floor or ceil of the problem's tiles / 8
    order = {t: i for i, t in enumerate(sorted(_expected_tiles(probs), key=lambda t: (t[0], t[1] // 4, t[2], t[1])))}
    for pi in range(len(probs)):
        prev_end, sizes = -1, []
        for q in range(nq):
            pos = sorted(order[t] for t in got[offsets[q]:offsets[q + 1]] if t[0] == pi)
            sizes.append(len(pos))
            if pos:
                assert pos == list(range(pos[0], pos[-1] + 1)) and pos[0] > prev_end, f"problem {pi} queue {q} band"
                prev_end = pos[-1]
        assert max(sizes) - min(sizes) <= 1, (pi, sizes)
    for q in range(nq):
        kt = ktiles[offsets[q]:offsets[q + 1]]
        assert np.all(np.diff(kt) <= 0), f"queue {q} is not longest-first"


def _sim(costs, cus):
    """List scheduling as the dispatcher does it: each item starts on the CU that frees first."""
    free = [0] * cus
    for c in costs:
        i = min(range(cus), key=free.__getitem__)
        free[i] += c
    return max(free)


def test_tail_tiles_split_into_halves_when_the_last_round_is_short():
    """C5's B X launch: 3200 equal tiles, 400 per queue on 32 CUs per XCD = 12
    rounds + 16 tiles.  With the CU count the last 16 tiles of every queue
    become 32 halves (12.5 rounds of work instead of 13); each half pair covers
    its tile exactly once and the halves come last in their queue."""
    probs = _lib.gemm_problems(_c5_phases()[2])
    items, offsets, n_wg, _ = _lib.gemm_schedule(probs, 32)
    p, tm, tn, part = _decode(items.astype(np.int64))
    nq = _lib.GEMM_QUEUES
    whole = set(zip(p[part == 0].tolist(), tm[part == 0].tolist(), tn[part == 0].tolist()))
    upper = list(zip(p[part == 1].tolist(), tm[part == 1].tolist(), tn[part == 1].tolist()))
    lower = list(zip(p[part == 2].tolist(), tm[part == 2].tolist(), tn[part == 2].tolist()))
    assert np.all(part < 3) and sorted(upper) == sorted(lower) and len(set(upper)) == len(upper)
    assert whole.isdisjoint(upper) and whole | set(upper) == _expected_tiles(probs)
    kt, epi = 4096 // _lib.GEMM_KTILE, 2 * 2
    for q in range(nq):
        qp = part[offsets[q]:offsets[q + 1]]
        assert (qp > 0).sum() == 32, q                         # 16 tiles -> 32 halves
        assert np.all(np.diff((qp > 0).astype(int)) >= 0), q   # halves last
        costs = [20 * (kt + epi) if x == 0 else 11 * kt + 10 * epi for x in qp.tolist()]
        assert _sim(costs, 32) < _sim([20 * (kt + epi)] * 400, 32)
    assert n_wg == nq * np.diff(offsets).max() == nq * (384 + 32)
    # a launch whose rounds are already full keeps whole tiles: 256 equal tiles per queue on 32 CUs
    full = _lib.gemm_problems(_ns_problems(4096, 4096 * 8, 1, 1 << 40)[2])
    items, _, _, _ = _lib.gemm_schedule(full, 32)
    assert np.all(_decode(items.astype(np.int64))[3] == 0)


def test_symmetric_tail_halves_keep_the_diagonal_unmirrored():
    """A small symmetric launch on few CUs: halves of diagonal and
    off-diagonal tiles both appear, and every tile on or above the diagonal is
    covered once (the kernel mirrors only off-diagonal tiles)."""
    probs = _lib.gemm_problems(_ns_problems(512, 512, 1, 1 << 40)[0])
    items, offsets, n_wg, _ = _lib.gemm_schedule(probs, 4)
    p, tm, tn, part = _decode(items.astype(np.int64))
    assert sorted(zip(tm[part == 1].tolist(), tn[part == 1].tolist())) == \
        sorted(zip(tm[part == 2].tolist(), tn[part == 2].tolist()))
    cover = {(a, b) for a, b, x in zip(tm.tolist(), tn.tolist(), part.tolist())}
    assert cover == {(0, 0), (0, 1), (1, 1)} and (part > 0).any()
    assert np.all(tm <= tn)


def test_schedule_symmetric_tile_count():
    probs = _ns_problems(1024, 1024, 1, 1 << 40)[0]
    items, offsets, _, _ = _lib.gemm_schedule(_lib.gemm_problems(probs))
    assert len(items) == 4 * 5 // 2                    # 4 x 4 tiles -> 10 on or above the diagonal


def test_schedule_rejects_invalid_problems():
    lib = _lib.load()
    good = _ns_problems(512, 768, 1, 1 << 40)

    def status(rows):
        arr = _lib.gemm_problems([tuple(r) for r in rows])
        n = lib.apexw_gemm_grouped_items(arr.ctypes.data, len(arr))
        return int(-n) if n < 0 else 0

    for rows in good:
        assert status(rows) == 0
    xx, aa, bx = (list(map(list, g)) for g in good)
    bad = [list(bx[0]) for _ in range(1)]
    bad[0][5] = 500                                       # m not a tile multiple
    assert status(bad) == 1
    bad = [list(bx[0])]
    bad[0][7] = 100                                       # k not a K-tile multiple
    assert status(bad) == 1
    bad = [list(xx[0])]
    bad[0][1] += 1 << 20                                  # symmetric product with a != b
    assert status(bad) == 1
    bad = [list(xx[0])]
    bad[0][4] += 1 << 20                                  # symmetric product with ct != c
    assert status(bad) == 1
    bad = [list(bx[0])]
    bad[0][0] += 2                                        # misaligned operand
    assert status(bad) == 4
    bad = [list(bx[0])]
    bad[0][8] = 512 + 4                                   # leading dimension not a multiple of 8
    assert status(bad) == 4
    bad = [list(bx[0])]
    bad[0][8] = 256                                       # lda < k
    assert status(bad) == 1
    bad = [list(bx[0])]
    bad[0][9] = 512                                       # [k x n] B with ldb < n
    assert status(bad) == 1
    bad = [list(bx[0])]
    bad[0][16] = 1                                        # reserved field
    assert status(bad) == 1
    bad = [list(aa[0])]
    bad[0][2] = 0                                         # beta != 0 without an addend
    assert status(bad) == 1
    bad = [list(bx[0])]
    bad[0][13] = 2.0                                      # addend from B needs alpha == 1
    assert status(bad) == 1
    bad = [list(bx[0])]
    bad[0][2] = bad[0][0]                                 # addend from B takes no et
    assert status(bad) == 1
    bad = [list(bx[0])]
    bad[0][4] = bad[0][3] + (1 << 20)                     # [k x n] B writes no transposed output
    assert status(bad) == 1
    bad = [list(xx[0])]
    bad[0][15] |= _lib.GEMM_B_KN                          # symmetric product with [k x n] B
    assert status(bad) == 1
    bad = [list(bx[0])]
    bad[0][5], bad[0][6], bad[0][7] = 768, 512, 512       # addend from B needs m <= k
    bad[0][8], bad[0][9], bad[0][11] = 512, 512, 512
    assert status(bad) == 1
    assert status([bx[0]] * 257) == 1                     # more problems than the item code holds
    # the fused Muon update (X' product only): p, dtype, shape within O, alignment
    A = _lib.GEMM_APPLY
    ok = list(bx[0]) + [1 << 41, 1, 512, 768, 0.99, -0.01, 0]
    ok[15] |= A | _lib.GEMM_APPLY_WD
    ok[3] = 0                                             # no X' store: the update is the only output
    assert status([ok]) == 0
    t = list(ok)
    t[15] |= _lib.GEMM_APPLY_T
    t[19], t[20] = 768, 512                               # p^T = O [512 x 768]
    assert status([t]) == 0
    t[19], t[20] = 512, 768                               # p^T would be 768 x 512: not covered by O
    assert status([t]) == 1
    bad = list(ok)
    bad[17] = 0                                           # no parameter
    assert status([bad]) == 1
    bad = list(ok)
    bad[18] = 7                                           # not a float dtype
    assert status([bad]) == 2
    bad = list(ok)
    bad[19] = 513                                         # more rows than O
    assert status([bad]) == 1
    bad = list(ok)
    bad[17] += 2                                          # fp32 parameter off its 4-byte alignment
    bad[18] = 0
    assert status([bad]) == 4
    bad = list(xx[0]) + [1 << 41, 1, 512, 512, 1.0, -0.01, 0]
    bad[15] |= A                                          # a symmetric product applies nothing
    assert status([bad]) == 1
    bad = list(bx[0]) + [1 << 41, 1, 512, 768, 0.0, -0.01, 0]
    assert status([bad]) == 1                             # update fields without the flag
    # a launch mixes no epilogue kinds
    arr = _lib.gemm_problems([tuple(xx[0]), tuple(bx[0])])
    with pytest.raises(_lib.ApexwError):
        _lib.gemm_schedule(arr)
    # the launch itself rejects bad kinds and null tables before enqueueing anything
    assert lib.apexw_gemm_nt_grouped(None, None, None, 16, 3, None, None) == 1
    assert lib.apexw_gemm_nt_grouped(16, 16, 16, 16, 4, None, None) == 1     # no output in the kind
    assert lib.apexw_gemm_nt_grouped(16, 16, 16, 12, 3, None, None) == 1     # grid not a multiple of the queues
    assert lib.apexw_gemm_nt_grouped(16, 16, 16, 16, 2 | 8, None, None) == 1  # [k x n] B with a transposed output
    assert lib.apexw_gemm_nt_grouped(16, 18, 16, 16, 3, None, None) == 4     # misaligned table


def test_panel_layout_flag():
    """APEXW_GEMM_PANEL: the launch's epilogue kind carries it (the kernel takes the
    layout at compile time), leading dimensions must be multiples of 32, a launch
    holds one layout, and the layout arguments of prepare / apply are checked."""
    lib = _lib.load()
    P = _lib.GEMM_PANEL
    for phase, rows in enumerate(_ns_problems(512, 1024, 2, 1 << 40)):
        panel = [tuple(r[:15]) + (r[15] | P, 0) for r in rows]
        *_, kind_rows = _lib.gemm_schedule(_lib.gemm_problems(rows))
        *_, kind_panel = _lib.gemm_schedule(_lib.gemm_problems(panel))
        assert kind_panel == kind_rows | _lib.GEMM_KIND_PANEL, phase
        # one layout per launch
        with pytest.raises(_lib.ApexwError):
            _lib.gemm_schedule(_lib.gemm_problems([panel[0], rows[1]]))
    # leading dimensions: multiples of 8 row-major, of 32 in panels
    x, a, nx = 1 << 40, 2 << 40, 3 << 40
    ok = _prob(a, x, 0, nx, 0, 512, 1024 + 256, 512, 520, 1288, 0, 1288, 0, 1.0, NS_A,
               _lib.GEMM_B_KN | _lib.GEMM_ADD_B)
    assert lib.apexw_gemm_grouped_items(_lib.gemm_problems([ok]).ctypes.data, 1) > 0
    bad = ok[:15] + (ok[15] | P, 0)
    assert lib.apexw_gemm_grouped_items(_lib.gemm_problems([bad]).ctypes.data, 1) == -4   # ld 520 / 1288
    # the launch accepts the panel bit in its kind, nothing above it
    assert lib.apexw_gemm_nt_grouped(16, 16, 16, 16, 32 | 1, None, None) == 1
    # prepare / apply: unknown layouts, and panels need ld % 32 == 0 (all pointers are
    # stand-ins: each call fails validation before anything is launched)
    st = lib.apexw_muon_prepare(16, 16, _lib.BF16, 300, 700, 0.9, 0.1, 0, 1e-7, 1.0, 16, None, 768, 0, 2, 16,
                                None, None)
    assert st == 1
    st = lib.apexw_muon_prepare(16, 16, _lib.BF16, 300, 700, 0.9, 0.1, 0, 1e-7, 1.0, 16, None, 712, 0,
                                _lib.LAYOUT_PANEL, 16, None, None)
    assert st == 4
    st = lib.apexw_muon_apply(16, _lib.BF16, 16, 300, 700, 712, _lib.LAYOUT_PANEL, 0, 0.99, 1, -0.01, None, None)
    assert st == 4
    st = lib.apexw_muon_apply(16, _lib.BF16, 16, 300, 700, 768, 5, 0, 0.99, 1, -0.01, None, None)
    assert st == 1


def test_panel_helpers_follow_the_documented_offsets():
    """NSWorkspace's row-major <-> panel conversions place element (r, c) of a
    matrix with ld columns at (r // 32) * 32 * ld + (c // 32) * 1024 + (r % 32) * 32
    + c % 32, the offset include/apexw_hip.h documents for APEXW_GEMM_PANEL, and
    invert each other."""
    import torch
    from apexw_amd.muon import _from_panels, _to_panels
    R, C = 96, 160
    t = torch.arange(R * C, dtype=torch.float32).view(R, C)
    p = _to_panels(t).reshape(-1)
    r = torch.arange(R).view(-1, 1).expand(R, C)
    c = torch.arange(C).view(1, -1).expand(R, C)
    off = (r // 32) * 32 * C + (c // 32) * 1024 + (r % 32) * 32 + c % 32
    assert torch.equal(p[off.reshape(-1)].view(R, C), t)
    assert torch.equal(_from_panels(_to_panels(t)), t)
    # a whole 32 x 32 panel is 1024 contiguous elements: rows 32..63, columns 64..95
    assert torch.equal(p[(1 * 5 + 2) * 1024:(1 * 5 + 3) * 1024].view(32, 32), t[32:64, 64:96])
