"""CPU model of the streamed expert GEMM's ring protocol (stream_gemm_kernel),
for the default consumers and the prefetching ones
(GPTOSS_MOE_FLAG_STAGE_PREFETCH).

The model walks the kernel's control flow stage by stage in "phases": phase
b is the time between barrier b and barrier b + 1 (phase -1 precedes barrier
0).  It records, per ring slot, when a producer issues the loads of a stage,
when the issuing wave has waited for them to land, and when a consumer reads
them and when those reads have returned.  It then checks, for every stage
and ring:

* a consumer reads a stage only after the barrier that follows its
  producer's landing wait (no read of bytes still in flight);
* the producer issues the stage that next occupies a slot only in a phase
  after every read of the slot's current stage has returned (no overwrite of
  a slot a consumer may still read);
* each consumer k step uses the register set holding that stage's k step;
* each lgkmcnt wait of the prefetching consumer covers its set: LDS returns
  in issue order, so after lgkmcnt(n) every operation except the last n
  issued has returned.

The control flow restated here follows the kernel's: s_consume_pre /
s_item_pre / s_stage_pre / s_read_k / s_wait_set for the prefetching
consumers, the s_barrier_mem loop for the default ones, and the producers'
prologue, `counted` landing wait and refill after each barrier."""
import random

import pytest

def stages_of(items, KP):
    """The workgroup's stage sequence: (item index, kp, units, row groups)."""
    out = []
    for i, (rows, cnt) in enumerate(items):
        for kp in range(KP):
            out.append((i, kp, cnt, (rows + 15) // 16))
    return out


def producer_schedule(S, depth, pre):
    """Issue phase and landing-wait phase of every stage for one producer
    wave: the prologue issues depth - 1 stages before barrier 0; before
    barrier s the wave waits for stages <= s (<= s + 1 with the prefetching
    consumers); after barrier s it issues the next stage."""
    issue, landed = {}, {}
    is_ = 0
    while is_ < depth - 1 and is_ < S:
        issue[is_] = -1
        is_ += 1
    counted = 0
    for s in range(S):
        assert s < is_
        while counted <= (s + 1 if pre else s) and counted < is_:
            landed[counted] = s - 1  # waited in the phase before barrier s
            counted += 1
        # barrier s
        if is_ < S:
            issue[is_] = s
            is_ += 1
    assert sorted(issue) == list(range(S)) and sorted(landed) == list(range(S))
    return issue, landed


class LdsQueue:
    """One consumer wave's LDS operations (in-order return)."""

    def __init__(self):
        self.ops = 0        # operations issued so far
        self.last_of = {}   # set tag -> index of its last operation

    def read(self, tag, n):
        if n:
            self.ops += n
            self.last_of[tag] = self.ops

    def wait_covers(self, tag, n):
        """After lgkmcnt(n), has set `tag` returned?"""
        return self.ops - self.last_of[tag] >= n


def consumer_pre(stages, KP, half, c, always_two=False, CT=2, cross=True):
    """The prefetching consumer c: a list of (phase, stage) reads with the
    phase their data is used in (returned by then), and the k steps it
    computes; asserts set contents and lgkmcnt coverage on the way."""
    reads = []          # (stage, read phase, used-by phase)
    computed = []
    sets = [None, None]
    q = LdsQueue()
    rd = 0
    s = 0
    phase = 0  # s_barrier_mem() before the first item: phase 0

    sc_of = [None, None]  # the stage whose e8m0 words a set holds

    def read_k(stage, ks, mt, p, ph):
        with_sc = ks < 2  # s_read_k<kSc>: only k steps 0, 1 read the e8m0 words
        n = (CT // 2) * (1 + with_sc) + mt if mt > 0 else 0
        if n:
            sets[p] = (stage, ks)
            if with_sc:
                sc_of[p] = stage
            q.read((stage, ks, p), n)
            reads.append((stage, ph))
        return n

    def use_set(p, stage, ks, rd_, ph):
        assert sets[p] == (stage, ks), (sets[p], stage, ks)
        assert sc_of[p] == stage, (sc_of[p], stage)
        n = CT // 2 + 1 if (rd_ > 0 or always_two) else 0  # s_min_ops
        assert q.wait_covers((stage, ks, p), n)
        computed.append((stage, ks, ph))

    while True:
        item, kp0, cnt, mt_rows = stages[s]
        assert kp0 == 0
        mt = mt_rows if (CT // 2) * c < cnt else 0
        if mt > 0:
            read_k(s, 0, mt, 0, phase)
            rd = read_k(s, 1, mt, 1, phase)
        # stages 0 .. KP - 2 (without cross: k steps 0, 1 read at each stage's
        # start, the next stage's not read ahead)
        for kp in range(KP - 1):
            if mt > 0:
                if not cross and kp > 0:
                    read_k(s, 0, mt, 0, phase)
                    rd = read_k(s, 1, mt, 1, phase)
                for j in range(4):
                    use_set(j & 1, s, j, rd, phase)
                    if j < 2:
                        rd = read_k(s, j + 2, mt, j & 1, phase)
                    else:
                        rd = read_k(s + 1, j - 2, mt if cross else 0, j & 1, phase)
            s += 1
            phase += 1  # barrier
        # last stage
        nks = 2 if half else 4
        if mt > 0:
            if not cross and KP > 1:
                read_k(s, 0, mt, 0, phase)
                rd = read_k(s, 1, mt, 1, phase)
            for j in range(nks):
                use_set(j & 1, s, j, rd, phase)
                if nks == 4 and j < 2:
                    rd = read_k(s, j + 2, mt, j & 1, phase)
                else:
                    rd = read_k(s + 1, j - (nks - 2), 0, j & 1, phase)
            reads.append((s, phase))  # the epilogue's bias / slot reads
        s += 1
        if s >= len(stages):
            break
        phase += 1
    assert s == len(stages) and phase == len(stages) - 1
    return reads, computed


def consumer_default(stages, c):
    """The default consumer: stage s's operands are read and used after
    barrier s."""
    reads = []
    for s, (_, _, cnt, _) in enumerate(stages):
        if c < cnt:
            reads.append((s, s))
    return reads


def check_ring(stages, reads_with_use, issue, landed, depth, pre):
    """Every read of stage t (read in phase r, used by phase u): landed
    before the barrier that opens phase r; the stage t + depth that next
    occupies its slot issued in a phase after u."""
    S = len(stages)
    for t, r, u in reads_with_use:
        assert landed[t] < r, (t, landed[t], r)
        nxt = t + depth
        if nxt < S:
            assert issue[nxt] > u, (t, r, u, issue[nxt])


def random_items(rng, KP, R=64):
    n = rng.randint(1, 6)
    return [(rng.randint(1, R), rng.randint(1, 8)) for _ in range(n)]


# (consumer kind, tile rows): the default consumers and the prefetching ones
# with 2 or 4 column tiles per wave; rings 5 / 4 deep for 64-row tiles, 3 / 3
# for 128-row tiles (SDepth)
KINDS = [(0, 64), (0, 128), (2, 64), (4, 64), (4, 128)]


@pytest.mark.parametrize("seed", range(30))
@pytest.mark.parametrize("kind,R", KINDS)
def test_ring_protocol(seed, kind, R):
    pre = kind != 0
    CT = kind or 2
    rng = random.Random(seed * 7 + kind + R)
    KP = rng.choice([1, 2, 3, 23])
    half = rng.random() < 0.5 and KP > 0
    items = random_items(rng, KP, R)
    stages = stages_of(items, KP)
    cross = pre and R == 64  # SKind::cross: read ahead across stages on 64-row tiles only
    for depth in ((5, 4) if R == 64 else (3,)):
        issue, landed = producer_schedule(len(stages), depth, cross)
        for c in range(16 // CT):
            if pre:
                reads, _ = consumer_pre(stages, KP, half, c, CT=CT, cross=cross)
                # a read is used by the end of the phase after it at the latest
                # (k steps 0, 1 of the next stage), else in its own phase
                with_use = []
                for t, ph in reads:
                    with_use.append((t, ph, t if t > ph else ph))
                check_ring(stages, with_use, issue, landed, depth, pre)
            else:
                reads = consumer_default(stages, c)
                check_ring(stages, [(t, r, r) for t, r in reads], issue, landed, depth, pre)


@pytest.mark.parametrize("seed", range(20))
@pytest.mark.parametrize("CT,R", [(2, 64), (4, 64), (4, 128)])
def test_prefetch_computes_every_k_step_once(seed, CT, R):
    rng = random.Random(1000 + seed)
    KP = rng.choice([1, 2, 5, 23])
    half = rng.random() < 0.5
    items = random_items(rng, KP, R)
    stages = stages_of(items, KP)
    units = [0] * 8
    for c in range(16 // CT):
        _, computed = consumer_pre(stages, KP, half, c, CT=CT, cross=R == 64)
        want = []
        for s, (_, kp, cnt, _) in enumerate(stages):
            if (CT // 2) * c < cnt:
                nks = 2 if (half and kp == KP - 1) else 4
                want += [(s, j) for j in range(nks)]
        assert [(s, j) for s, j, _ in computed] == want
        # a stage's k steps are computed in its own phase
        assert all(ph == s for s, _, ph in computed)


def test_two_deep_ring_would_read_uncertified_bytes():
    # the landing wait for stage s + 1 before barrier s needs that stage
    # issued by then, which holds from a 3-deep ring up (both rings here are
    # 4 and 5 deep); with 2 the model must flag the prefetch
    stages = stages_of([(40, 8)], 6)
    for depth in (3, 4, 5):
        issue, landed = producer_schedule(len(stages), depth, True)
        reads, _ = consumer_pre(stages, 6, True, 0)
        check_ring(stages, [(t, ph, t if t > ph else ph) for t, ph in reads], issue, landed, depth, True)
    issue, landed = producer_schedule(len(stages), 2, True)
    reads, _ = consumer_pre(stages, 6, True, 0)
    with pytest.raises(AssertionError):
        check_ring(stages, [(t, ph, t if t > ph else ph) for t, ph in reads], issue, landed, 2, True)


def test_model_flags_an_unshifted_producer_wait():
    # prefetching consumers against producers that wait for stage s only
    # before barrier s: the model must flag the read of stage s + 1
    stages = stages_of([(40, 8), (20, 3)], 5)
    issue, landed = producer_schedule(len(stages), 5, False)
    reads, _ = consumer_pre(stages, 5, True, 0)
    with pytest.raises(AssertionError):
        check_ring(stages, [(t, ph, t if t > ph else ph) for t, ph in reads], issue, landed, 5, True)


def test_model_flags_lgkmcnt2_without_a_later_set():
    # the last k step of an item has no later set in flight: lgkmcnt(2) there
    # would not cover it
    stages = stages_of([(40, 8)], 3)
    consumer_pre(stages, 3, False, 0)
    with pytest.raises(AssertionError):
        consumer_pre(stages, 3, False, 0, always_two=True)


@pytest.mark.parametrize("CT", [2, 4])
def test_every_weight_unit_has_one_consumer(CT):
    """Consumer c owns weight units (CT / 2) c .. (CT / 2) c + CT / 2 - 1 of an
    item (the epilogue skips units >= cnt): each of the item's units once."""
    for cnt in range(1, 9):
        owned = []
        for c in range(16 // CT):
            for h in range(CT // 2):
                u = (CT // 2) * c + h
                if u < cnt:
                    owned.append(u)
        assert sorted(owned) == list(range(cnt))


def test_model_flags_a_one_stage_lookahead_on_3_deep_rings():
    # reading ahead across stages (producers waiting one stage earlier) on
    # a 3-deep ring would still be correct, but leaves the producers only one
    # stage of lookahead; the kernel does not do it (SKind::cross), and the
    # model of the kernel's choice keeps two: issue of stage t at least two
    # barriers before the barrier that certifies it
    stages = stages_of([(100, 8), (60, 5)], 6)
    issue, landed = producer_schedule(len(stages), 3, False)
    assert all(landed[t] - issue[t] >= 1 for t in range(3, len(stages)))
    issue, landed = producer_schedule(len(stages), 3, True)
    assert any(landed[t] - issue[t] < 1 for t in range(3, len(stages)))
