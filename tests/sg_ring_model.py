"""State-machine model of the SG list ring protocol between GPU submitter
waves and transfer waves (include/gfd/sg_device_primitives.h,
include/gfd/sg_warp_spec.h; the reference's protocol is
include/gfd/sg_device_primitives.cuh:27-242 and sg_warp_spec.cuh:95-261).
Test infrastructure: the CPU tests explore it, nothing ships it.

Shared state, as in the kernels:
- list_alloc, list_claim, list_known, lists_done, stop, terminate: HBM
  counters and words (SGDeviceCounters, SGTaskQueue::terminate);
- seq[s], done[s]: ring slot s's `sequence` and `done` words in host memory.

Submitter wave (one per workgroup), for each of its lists:
  space   wait until list_alloc - lists_done < R - 1   (sg_wait_list_space)
  alloc   slot = list_alloc++                           (sg_alloc_list)
  slot    wait until done[slot % R] >= slot - R + 1     (sg_wait_slot_free)
  commit  seq[slot % R] = slot + 1, a release           (sg_commit_list)
With place "fixed" (the MoE kernel when the launch's lists fit the ring:
total < R), list L goes to ring index L with no space, allocation or slot
wait: the submitter commits seq[L % R] = L + 1 directly.
stop "wait": submitter 0 then waits until lists_done == total and raises
terminate and stop (sg_wait_gpu_lists_done + sg_terminate_all_landed).
stop "lander" (sg_stop_when_landed): submitter 0 sets stop_at = total and,
if lists_done >= total already, raises them itself; the transfer wave whose
landing brings lists_done to stop_at raises them otherwise (each of these
steps is one atomic move here, as the kernels make them sequentially
consistent).  Lists reach the submitters either as the MoE kernel deals
them (list L to submitter L mod S, each in order: "mod") or from a shared
counter ("shared": the variant that was tried and taken out).

Transfer wave, per list:
  claim   idx = list_claim++
  wait    _wait_committed's list_known protocol: a wave whose idx is below
          list_known goes on; the wave at list_known (the leader) reads
          terminate, then seq; when its list is committed it finds the run
          of committed indices from idx (up to R of them) and raises
          list_known past it; when terminate was set it raises stop and
          exits; any wave exits once stop is set
  read    the header is read; the claim store seq[idx % R] = 0
  land    done[idx % R] = idx + 1, a system-scope release; lists_done++
          (stop "lander": then terminate and stop if lists_done reached a
          nonzero stop_at)

claim_store "ordered": the claim store is performed before the release of
done (a store followed by a release in the same wave).  "reorderable": it
may be performed at any later point, after done included (a claim store
with no order against the release).

A state in which no wave can move is a deadlock unless every list landed
exactly once and every wave has ended.  Waits never time out in the model,
so a deadlock here is a launch that only a time limit would end.
"""
import random
from collections import deque

SPACE, ALLOC, SLOT, COMMIT, NEXT, FINAL, END = range(7)  # submitter
CLAIM, WAIT, READ, LAND, WEND = range(5)                 # transfer wave


class State:
    __slots__ = ("la", "lc", "lk", "ld", "stop", "term", "nid", "sa", "seq", "done", "landed", "subs", "waves")

    def clone(self):
        s = State.__new__(State)
        s.la, s.lc, s.lk, s.ld, s.stop, s.term, s.nid = self.la, self.lc, self.lk, self.ld, self.stop, self.term, self.nid
        s.sa = self.sa
        s.seq, s.done, s.landed = list(self.seq), list(self.done), list(self.landed)
        s.subs, s.waves = [list(x) for x in self.subs], [list(x) for x in self.waves]
        return s

    def key(self):
        return (self.la, self.lc, self.lk, self.ld, self.stop, self.term, self.nid, self.sa, tuple(self.seq), tuple(self.done),
                tuple(self.landed), tuple(map(tuple, self.subs)), tuple(map(tuple, self.waves)))


class Model:
    def __init__(self, ring, submitters, waves, total, assign="mod", claim_store="ordered", place="alloc",
                 stop="wait"):
        assert assign in ("mod", "shared") and claim_store in ("ordered", "reorderable")
        # "lander_unchecked": a planted mistake for the tests, submitter 0
        # setting stop_at without checking whether every list has landed.
        assert place in ("alloc", "fixed") and stop in ("wait", "lander", "lander_unchecked")
        assert place == "alloc" or total < ring, "fixed places need the launch's lists to fit the ring"
        self.R, self.S, self.W, self.total = ring, submitters, waves, total
        self.assign, self.claim_store, self.place, self.stop = assign, claim_store, place, stop

    def initial(self):
        s = State()
        s.la = s.lc = s.lk = s.ld = s.stop = s.term = s.nid = s.sa = 0
        s.seq, s.done, s.landed = [0] * self.R, [0] * self.R, [0] * self.total
        s.subs = [[NEXT, -1, k, -1] for k in range(self.S)]  # pc, list, next own list (mod), slot
        s.waves = [[CLAIM, -1, -1] for _ in range(self.W)]   # pc, idx, slot of a claim store in flight
        return s

    def step_sub(self, s, i):
        """One step of submitter i, in place; False if it cannot move."""
        sub, R = s.subs[i], self.R
        pc = sub[0]
        if pc == NEXT:
            if self.assign == "mod":
                sub[1], sub[2] = sub[2], sub[2] + self.S
            else:
                sub[1], s.nid = s.nid, s.nid + 1
            if sub[1] >= self.total:
                sub[0] = FINAL if i == 0 else END
            elif self.place == "fixed":
                sub[3], sub[0] = sub[1], COMMIT
            else:
                sub[0] = SPACE
        elif pc == SPACE:
            if s.la - s.ld >= R - 1:
                return False
            sub[0] = ALLOC
        elif pc == ALLOC:
            sub[3], s.la, sub[0] = s.la, s.la + 1, SLOT
        elif pc == SLOT:
            slot = sub[3]
            if slot >= R and s.done[slot % R] < slot - R + 1:
                return False
            sub[0] = COMMIT
        elif pc == COMMIT:
            s.seq[sub[3] % R] = sub[3] + 1
            sub[0], sub[3] = NEXT, -1
        elif pc == FINAL:
            if self.stop in ("lander", "lander_unchecked"):
                s.sa = self.total
                if self.stop == "lander" and s.ld >= self.total:
                    s.term, s.stop = 1, 1
                sub[0] = END
                return True
            if s.ld < self.total:
                return False
            s.term, s.stop, sub[0] = 1, 1, END
        else:
            return False
        return True

    def step_wave(self, s, j, flush=False):
        """One step of transfer wave j, or (flush) the late claim store of a
        reorderable one, in place; False if it cannot move."""
        w, R = s.waves[j], self.R
        if flush:
            if w[2] < 0:
                return False
            s.seq[w[2]] = 0
            w[2] = -1
            return True
        pc, idx = w[0], w[1]
        if pc == CLAIM:
            w[1], s.lc, w[0] = s.lc, s.lc + 1, WAIT
        elif pc == WAIT:
            if idx < s.lk:
                w[0] = READ
            elif idx == s.lk:
                term = s.term  # read before the sequence
                if s.seq[idx % R] == idx + 1:
                    run = 0
                    while run < R and s.seq[(idx + run) % R] == idx + run + 1:
                        run += 1
                    s.lk, w[0] = max(s.lk, idx + run), READ
                elif term:
                    s.stop, w[0] = 1, WEND
                elif s.stop:
                    w[0] = WEND
                else:
                    return False
            else:
                if not s.stop:
                    return False
                w[0] = WEND
        elif pc == READ:
            if self.claim_store == "ordered":
                s.seq[idx % R] = 0
            else:
                if w[2] >= 0:  # one claim store in flight per wave
                    return False
                w[2] = idx % R
            w[0] = LAND
        elif pc == LAND:
            if self.claim_store == "ordered" and w[2] >= 0:
                return False
            s.done[idx % R] = idx + 1
            if idx < self.total:
                s.landed[idx] += 1
            s.ld += 1
            if self.stop != "wait" and s.sa and s.ld >= s.sa:
                s.term, s.stop = 1, 1
            w[0], w[1] = CLAIM, -1
        else:
            return False
        return True

    def moves(self):
        """Every actor step: (kind, index, flush)."""
        out = [("s", i, False) for i in range(self.S)]
        out += [("w", j, False) for j in range(self.W)]
        if self.claim_store == "reorderable":
            out += [("w", j, True) for j in range(self.W)]
        return out

    def apply(self, s, move):
        kind, i, flush = move
        return self.step_sub(s, i) if kind == "s" else self.step_wave(s, i, flush)

    def finished_ok(self, s):
        return (all(x[0] == END for x in s.subs) and all(w[0] == WEND and w[2] < 0 for w in s.waves)
                and all(c == 1 for c in s.landed))

    def explore(self, max_states=3_000_000):
        """Every interleaving, breadth first.  Returns (states, problem):
        problem is None, or (kind, moves) with the moves from the initial
        state to a state that is stuck or has landed a list twice."""
        start = self.initial()
        k0 = start.key()
        parent = {k0: None}
        q = deque([(start, k0)])
        moves = self.moves()
        while q:
            s, k = q.popleft()
            if any(c > 1 for c in s.landed):
                return len(parent), ("list landed twice", self._path(parent, k))
            moved = False
            for m in moves:
                n = s.clone()
                if not self.apply(n, m):
                    continue
                moved = True
                nk = n.key()
                if nk not in parent:
                    parent[nk] = (k, m)
                    if len(parent) > max_states:
                        raise RuntimeError("state space larger than %d" % max_states)
                    q.append((n, nk))
            if not moved and not self.finished_ok(s):
                return len(parent), ("deadlock", self._path(parent, k))
        return len(parent), None

    @staticmethod
    def _path(parent, k):
        path = []
        while parent[k] is not None:
            k, m = parent[k]
            path.append(m)
        return path[::-1]

    def simulate(self, seed, skew=True, max_steps=20_000_000):
        """One random interleaving.  With skew, each actor gets a speed drawn
        log-uniformly over three decades and moves that often relative to
        the others (one slow submitter or transfer wave among fast ones).
        Returns (steps, outcome): "ok", "deadlock" or "list landed twice"."""
        rng = random.Random(seed)
        s = self.initial()
        moves = self.moves()
        speed = {}
        for m in moves:
            who = m[:2]
            if who not in speed:
                speed[who] = 10.0 ** rng.uniform(-3, 0) if skew else 1.0
        weights = [speed[m[:2]] for m in moves]
        for step in range(max_steps):
            # Weighted order without replacement: the first move that can go, goes.
            order = sorted(range(len(moves)), key=lambda i: -rng.random() ** (1.0 / weights[i]))
            if not any(self.apply(s, moves[i]) for i in order):
                return step, "ok" if self.finished_ok(s) else "deadlock"
            if any(c > 1 for c in s.landed):
                return step, "list landed twice"
        raise RuntimeError("no end after %d steps" % max_steps)

    def replay(self, path):
        """The states along a path of moves, with what each move did."""
        s = self.initial()
        lines = []
        for m in path:
            assert self.apply(s, m)
            who = ("submitter %d" % m[1]) if m[0] == "s" else ("wave %d%s" % (m[1], " claim store" if m[2] else ""))
            lines.append("%-20s seq=%s done=%s known=%d alloc=%d claim=%d landed=%d" %
                         (who, s.seq, s.done, s.lk, s.la, s.lc, s.ld))
        return s, lines
