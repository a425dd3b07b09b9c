"""Host-side checks of the projection-chain schedule (sys1hip_linear_chain_bf16,
sys1_amd/csrc/chain.hip), without a device.

1. The per-XCD tile queues (the library's own decode, through
   sys1hip_chain_queue) partition every chain's tiles exactly once, each
   queue holds the row panels r with r % 8 == its XCD, and every tile's
   dependencies (the previous projection's tiles on its row panel) come
   earlier in its queue.
2. A model of one launch's wave protocol -- compute wave 0 taking tiles and
   publishing them with their readiness, the compute waves counting a tile
   a k-step into the next one (at once before a drain or the end), the
   producer waves' issue cursor,
   decision, drain and end, and the barriers both sides meet -- run under
   random interleavings of many workgroups on the real queues: every
   workgroup's producer and compute waves meet the same barriers in the same
   order, nothing deadlocks, no dependency wait has to give up, every tile is
   computed exactly once, a tile's first k-tile is issued only once its
   dependency is complete, and the compute waves read a stage only after its
   k-tile was issued.  The model restates the kernel's control flow step by
   step (the names follow the kernel's).
"""
import random

import pytest

from sys1_amd import _lib

STAGES = 3
BM, BN = 128, 192
WAVES = 8  # compute waves per workgroup (each releases its part of a tile)

CHAINS = {
    # name: [(N, K)] of the projections of one launch
    "modernbert-base": [(768, 768), (2304, 768), (768, 1152), (2304, 768)],
    "modernbert-large": [(1024, 1024), (5248, 1024), (1024, 2624), (3072, 1024)],
    "qwen-small-deltanet": [(2048, 4096), (12288, 2048), (2048, 6144), (12320, 2048)],
    "two": [(768, 768), (2304, 768)],
    "one": [(2304, 768)],
}


def _tiles(chain, M):
    return {(p, rp, tn) for p, (N, _) in enumerate(chain)
            for rp in range(-(-M // BM)) for tn in range(-(-N // BN))}


@pytest.mark.parametrize("name", sorted(CHAINS))
@pytest.mark.parametrize("M", [1, 127, 128, 129, 1000, 8050, 16384])
def test_queues_partition_the_tiles_in_dependency_order(name, M):
    chain = CHAINS[name]
    Ns = [n for n, _ in chain]
    seen = []
    for xcc in range(8):
        q = _lib.chain_queue(xcc, M, Ns)
        pos = {t: i for i, t in enumerate(q)}
        assert len(pos) == len(q)
        for (p, rp, tn) in q:
            assert rp % 8 == xcc
            if p > 0:
                deps = [pos[(p - 1, rp, j)] for j in range(-(-Ns[p - 1] // BN))]
                assert max(deps) < pos[(p, rp, tn)]
        seen += q
    assert len(seen) == len(set(seen)) and set(seen) == _tiles(chain, M)


class Launch:
    """Shared state of one launch: the queues, the dependency counters, the
    slots and barriers of every workgroup, and what was issued / read."""

    def __init__(self, chain, M, per_xcd, seed):
        self.chain = chain
        self.kt = [K // 64 for _, K in chain]
        self.tn = [-(-N // BN) for N, _ in chain]
        self.queues = [_lib.chain_queue(x, M, [n for n, _ in chain]) for x in range(8)]
        self.heads = [0] * 8
        self.deps = {}
        self.computed = []
        self.rng = random.Random(seed)
        self.wgs = [(x, g) for x in range(8) for g in range(per_xcd)]

    def grab(self, xcc):
        i = self.heads[xcc]
        self.heads[xcc] += 1
        return i if i < len(self.queues[xcc]) else -1

    def dep_met(self, xcc, i):
        p, rp, _ = self.queues[xcc][i]
        return p == 0 or self.deps.get((p - 1, rp), 0) >= self.tn[p - 1] * WAVES


def _compute(L, xcc, wg):
    """Compute waves (wave 0's taking and publishing included)."""
    q = L.queues[xcc]
    i = L.grab(xcc)
    if i >= 0 and not L.dep_met(xcc, i):
        yield ("wait", lambda: L.dep_met(xcc, i))
    wg["slot"][0] = (i, 1)
    yield ("bar", "init")
    first = wg["slot"][0][0]
    if first < 0:
        yield ("bar", "final")
        return
    ct = q[first]
    kc, ckt, n, s = L.kt[ct[0]], 0, 0, 0
    yield ("bar", "start")
    wg["read"].append(0)
    next_raw = next_id = -1
    poll = 0
    pending = None

    def release(t):
        L.deps[(t[0], t[1])] = L.deps.get((t[0], t[1]), 0) + WAVES

    while True:
        assert wg["issued"] > s, "a k-tile's fragments read before it was issued"
        rel_at = 1 if kc > STAGES + 1 else 0
        if pending is not None and ckt == rel_at:
            release(pending)
            pending = None
        if ckt == rel_at:
            next_raw = L.grab(xcc)
        if ckt == max(0, kc - STAGES - 1):
            next_id = next_raw
            if next_id >= 0 and q[next_id][0] > 0:
                p, rp, _ = q[next_id]
                poll = L.deps.get((p - 1, rp), 0)
        if ckt == kc - STAGES:
            ready = 1
            if next_id >= 0 and q[next_id][0] > 0:
                ready = int(poll >= L.tn[q[next_id][0] - 1] * WAVES)
            wg["slot"][(n + 1) % 4] = (next_id, ready)
        yield ("bar", ("s", s))
        last = ckt + 1 == kc
        nid, rdy = wg["slot"][(n + 1) % 4] if last else (0, 1)
        streamed = not last or (nid >= 0 and rdy)
        if streamed:
            assert wg["issued"] > s + 1, "next k-tile's first fragments read before it was issued"
        if not last:
            ckt, s = ckt + 1, s + 1
            continue
        L.computed.append(ct)
        if streamed:
            pending = ct  # counted a k-step into the next tile
        else:
            release(ct)
        if nid < 0:
            break
        if not streamed:
            yield ("bar", ("D", s))
            assert wg["issued"] > s + 1
        n += 1
        ct = q[nid]
        kc, ckt, s = L.kt[ct[0]], 0, s + 1
    yield ("bar", "final")


def _producer(L, xcc, wg):
    """Producer waves: the issue cursor, decisions, drains and the end."""
    q = L.queues[xcc]
    yield ("bar", "init")
    first = wg["slot"][0][0]
    if first < 0:
        yield ("bar", "final")
        return

    def issue_tile_start(i):
        assert L.dep_met(xcc, i), f"tile {q[i]} issued before its dependency was complete"

    it = first
    issue_tile_start(it)
    ikc = L.kt[q[it][0]]
    n, F_next, last_step, drain_at, next_id = 0, ikc, -1, -1, -1
    wg["issued"] = STAGES
    yield ("bar", "start")
    s = 0
    while True:
        yield ("bar", ("s", s))
        if s + STAGES == F_next and last_step < 0 and drain_at < 0:
            next_id, rdy = wg["slot"][(n + 1) % 4]
            if next_id < 0:
                last_step = F_next - 1
            elif not rdy:
                drain_at = F_next - 1
            else:
                n += 1
                it = next_id
                issue_tile_start(it)
                F_next += L.kt[q[it][0]]
        if s == last_step:
            break
        if s == drain_at:
            if not L.dep_met(xcc, next_id):
                nid_ = next_id
                yield ("wait", lambda: L.dep_met(xcc, nid_))
            n += 1
            it = next_id
            issue_tile_start(it)
            F_next += L.kt[q[it][0]]
            wg["issued"] = s + 1 + STAGES
            drain_at = -1
            yield ("bar", ("D", s))
            s += 1
            continue
        qs = s + STAGES
        if qs < F_next and wg["issued"] == qs:
            wg["issued"] = qs + 1
        s += 1
    yield ("bar", "final")


def _run(chain, M, per_xcd, seed):
    L = Launch(chain, M, per_xcd, seed)
    actors = []
    for xcc, g in L.wgs:
        wg = {"slot": [None] * 4, "issued": 0, "read": []}
        actors.append({"wg": wg, "gens": [_compute(L, xcc, wg), _producer(L, xcc, wg)],
                       "state": [None, None], "done": [False, False]})
    # advance each generator to its first yield
    for a in actors:
        for k in range(2):
            a["state"][k] = next(a["gens"][k])
    steps = 0
    while True:
        runnable = []
        for ai, a in enumerate(actors):
            st = a["state"]
            if all(a["done"]):
                continue
            if not a["done"][0] and not a["done"][1] and st[0][0] == "bar" and st[1][0] == "bar":
                assert st[0][1] == st[1][1], f"barrier mismatch: compute at {st[0][1]}, producers at {st[1][1]}"
                runnable.append((ai, None))
            for k in range(2):
                if not a["done"][k] and st[k][0] == "wait" and st[k][1]():
                    runnable.append((ai, k))
        if not runnable:
            break
        ai, k = L.rng.choice(runnable)
        a = actors[ai]
        for kk in ((0, 1) if k is None else (k,)):
            try:
                a["state"][kk] = next(a["gens"][kk])
            except StopIteration:
                a["done"][kk] = True
        steps += 1
        assert steps < 5_000_000
    stuck = [ai for ai, a in enumerate(actors) if not all(a["done"])]
    assert not stuck, f"deadlock: workgroups {stuck[:8]} never finished"
    assert sorted(L.computed) == sorted(_tiles(chain, M)), "tiles computed more or less than once"


@pytest.mark.parametrize("name", ["modernbert-base", "qwen-small-deltanet", "two", "one"])
@pytest.mark.parametrize("M,per_xcd,seeds", [(1, 4, 3), (129, 3, 3), (1000, 4, 3), (3000, 32, 1), (8050, 5, 1)])
def test_wave_protocol_under_random_interleavings(name, M, per_xcd, seeds):
    for seed in range(seeds):
        _run(CHAINS[name], M, per_xcd, seed)


def _swz(r):
    return (r ^ (r >> 3)) & 7


@pytest.mark.parametrize("name", sorted(CHAINS))
@pytest.mark.parametrize("M", [1, 129, 8050])
@pytest.mark.parametrize("blocked", [False, True])
def test_every_access_of_every_tile_stays_inside_its_operand(name, M, blocked):
    """The byte ranges the chain kernel touches for each tile of the queues,
    restated from its producer offsets (x and w refills, 16-byte chunks per
    lane, k-tile offsets) and its epilogue (16-byte stores and residual
    reads): every one inside its operand ([M, ldx] x, [N, ldw] or blocked w,
    [M, ldy] y, [M, ldr] residual) -- the host-side check that no launch of
    these shapes reads or writes outside the tensors it was given."""
    chain = CHAINS[name]
    Ns = [n for n, _ in chain]
    RPI, XT = 8, BM // 8            # rows per 1 KB DMA instruction, x instructions per k-tile
    DT = (BM + BN) // 8
    for xcc in range(8):
        for (p, rp, tn) in _lib.chain_queue(xcc, M, Ns):
            N, K = chain[p]
            ldx, ldw = K + 8, K + 16  # leading dimensions wider than K, as column slices have
            w_kt = -(-K // 64)
            m0, n0 = rp * BM, tn * BN
            assert m0 < M
            x_left, w_left = M - 1 - m0, N - 1 - n0
            x_hi = w_hi = 0
            # rows of the tile's x and w refills (instruction u covers RPI rows;
            # a lane's chunk is lpos ^ swz(row): every chunk 0..7 of each row)
            for u in range(DT):
                for lrow in range(RPI):
                    r = (u if u < XT else u - XT) * RPI + lrow
                    cmax = max(lpos ^ _swz(r) for lpos in range(8))
                    kt = K // 64 - 1
                    if u < XT:
                        x_hi = max(x_hi, (m0 * ldx + min(r, x_left) * ldx) * 2 + cmax * 16 + kt * 128 + 16)
                    else:
                        rw = min(r, w_left)
                        if blocked:
                            off = ((n0 // 32) * w_kt + (rw // 32) * w_kt + kt) * 4096 + (rw % 32) * 128 + cmax * 16
                        else:
                            off = (n0 * ldw + rw * ldw) * 2 + cmax * 16 + kt * 128
                        w_hi = max(w_hi, off + 16)
            assert x_hi <= ((M - 1) * ldx + K) * 2
            w_bytes = -(-N // 32) * w_kt * 4096 if blocked else ((N - 1) * ldw + K) * 2
            assert w_hi <= w_bytes
            # epilogue: rows m < M only, columns n < Nout only, 16 bytes each
            gated = name.startswith(("modernbert", "qwen")) and p == 1
            nout = N // 2 if gated else N
            ldy = ldr = nout + 8
            cols = range((n0 // 2 if gated else n0), min(nout, (n0 + BN) // 2 if gated else n0 + BN), 8)
            last_row = min(M, m0 + BM) - 1
            for n in cols:
                assert n + 8 <= nout
                assert (last_row * ldy + n + 8) * 2 <= ((M - 1) * ldy + nout) * 2


@pytest.mark.parametrize("M", [1, 17, 64])
@pytest.mark.parametrize("blocked", [False, True])
@pytest.mark.parametrize("name,chain", [
    ("modernbert-large", [(1024, 1024, "res"), (5248, 1024, "gated"), (1024, 2624, "res"), (3072, 1024, "none")]),
    ("modernbert-base", [(768, 768, "res"), (2304, 768, "gated"), (768, 1152, "res"), (2304, 768, "none")]),
    ("short-k", [(96, 64, "none"), (64, 40, "res")])])
def test_weight_streaming_chain_accesses_stay_inside_their_operands(M, blocked, name, chain):
    """The weight-streaming chain (up to 64 tokens: 32-column items over the
    whole K, K split over 12 waves of at most 7 k-steps of 32): every byte
    offset its loads and stores form, restated from the kernel -- weight rows
    clamped to N, token rows to M, k-chunks past K out of range, no negative
    k-step offset for a wave without k-steps -- lies inside the operand."""
    NW, SMAX, BN, BM = 12, 7, 32, 64
    OOR = 0x80000000
    for N, K, kind in chain:
        assert K <= SMAX * 32 * NW
        ldx, ldw = K + 8, K + 24
        w_kt = -(-K // 64)
        nout = N // 2 if kind == "gated" else N
        ldy = nout + 16
        ksteps = -(-K // 32)
        for cb in range(-(-N // BN)):
            n0 = cb * BN
            for wave in range(NW):
                s0, s1 = wave * ksteps // NW, (wave + 1) * ksteps // NW
                for lane in range(64):
                    r16, q = lane & 15, lane >> 4
                    for u in range(SMAX):
                        st = s0 + u
                        ok = st < s1 and st * 32 + q * 8 < K
                        sc = max(0, min(st, s1 - 1))
                        assert sc >= 0
                        if not ok:
                            continue  # out-of-range offset: no access
                        for i in range(2):
                            nr = min(n0 + i * 16 + r16, N - 1)
                            if blocked:
                                off = (nr // 32) * w_kt * 4096 + (nr % 32) * 128 + q * 16 + (sc >> 1) * 4096 + (sc & 1) * 64
                                assert off + 16 <= -(-N // 32) * w_kt * 4096
                            else:
                                off = nr * ldw * 2 + q * 16 + sc * 64
                                assert off + 16 <= ((N - 1) * ldw + K) * 2
                        for j in range(BM // 16):
                            xo = min(j * 16 + r16, M - 1) * ldx * 2 + q * 16 + sc * 64
                            assert xo + 16 <= ((M - 1) * ldx + K) * 2
            # epilogue: rows r < M, 8-column vectors n < Nout
            vecs = BN // 16 if kind == "gated" else BN // 8
            out_n0 = n0 // 2 if kind == "gated" else n0
            for t in range(BM * vecs):
                r, c0 = t // vecs, (t % vecs) * 8
                if r >= M or out_n0 + c0 >= nout:
                    continue
                assert (r * ldy + out_n0 + c0 + 8) * 2 <= ((M - 1) * ldy + nout) * 2
