"""CPU model of the one-launch backward's dQ hand-over (gpt_amd/csrc/
attn_bwd_fused_kernel.h: the schedule at the end of bwd_fused_d64_kernel), run
under adversarial schedules.

Main workgroups (one per key group J of a (b, h)) and orphan runners are
generators that yield after every access to the control block, in the
kernel's order:

* a main workgroup walks query blocks n_qb - 1 down to 2J, bumping each
  block's completion counter after its dS stores (a relaxed atomic: the
  scheduler may make a bump visible late); then thread 0 decides its own dQ
  item (blocks 2J + 1, 2J): key group 0 runs it at once (its tiles are its
  own), the others wait a bounded number of polls for both counters to
  reach J + 1, and if they are still short, store the item's orphan flag
  (the launch epoch) and wait for that store before adding 1 to the done
  counter; an item decided to run is run, then its counters are released;
* an orphan runner waits until the done counter of its (b, h) reaches the
  number of key groups, then runs every item flagged with this launch's
  epoch (waiting for its counts, which cannot be short any more), releasing
  the counters after each, and finally subtracts the key-group count from
  the done counter.

Main workgroups are dispatched in any order, the runners last (the grid's
highest indices; the hardware dispatches a launch's workgroups in index
order), and at most `resident` workgroups run at once. The model checks:

* no deadlock at any residency: owners' waits are bounded, and runners wait
  only for main workgroups, which never wait for runners;
* every dQ item runs exactly once, and (except item 0, which reads only its
  own workgroup's tiles) only after all of its contributions have landed;
* every launch leaves its counters and done counter at 0, and later
  launches (new epochs) work on the same control block without clearing it.

Two planted mistakes show that the checks catch what they are meant to: an
owner that waits without a bound (the earlier whole-grid-resident design)
deadlocks at low residency, and an orphan flag that becomes visible only
after the done counter moved is missed by the runners.
"""
import random

import pytest

OWNER_POLLS = 20  # an owner's bounded wait, in polls


class ControlBlock:
    """Counters, orphan flags and the done counter of one (b, h)."""

    def __init__(self, n_qb, n_kg):
        self.cnt = [0] * n_qb
        self.orphan = [0] * n_kg
        self.done = 0


def counts_ok(ctl, J, n_qb, need):
    return ctl.cnt[2 * J] >= need and (2 * J + 1 >= n_qb or ctl.cnt[2 * J + 1] >= need)


def release(ctl, J, n_qb):
    ctl.cnt[2 * J] -= J + 1
    if 2 * J + 1 < n_qb:
        ctl.cnt[2 * J + 1] -= J + 1


def main_wg(J, n_qb, ctl, epoch, log, state):
    for i in range(n_qb - 1, 2 * J - 1, -1):
        state["bumps"].append(i)
        yield
    run = True
    if J > 0:
        polls = 0
        while True:
            ok = counts_ok(ctl, J, n_qb, J + 1)
            yield "poll" if state["planted"] == "unbounded_owner" else None
            if ok:
                break
            polls += 1
            if polls > OWNER_POLLS and state["planted"] != "unbounded_owner":
                run = False
                break
        if not run:
            if state["planted"] == "late_flag":
                state["late_flags"].append((J, epoch))
            else:
                ctl.orphan[J] = epoch
            state["orphans"] += 1
            yield
    ctl.done += 1
    yield
    if run:
        log.append((J, counts_ok(ctl, J, n_qb, J + 1)))
        release(ctl, J, n_qb)
        yield


def runner(n_qb, ctl, epoch, log):
    n_kg = len(ctl.orphan)
    while ctl.done < n_kg:
        yield "poll"
    for J in range(n_kg):
        if ctl.orphan[J] != epoch:
            continue
        yield
        while not counts_ok(ctl, J, n_qb, J + 1):
            yield "poll"
        log.append((J, True))
        release(ctl, J, n_qb)
        yield
    ctl.done -= n_kg
    yield


def run_launch(n_qb, resident, seed, ctl, epoch, planted=None, max_events=400000):
    rng = random.Random(seed)
    n_kg = (n_qb + 1) // 2
    log = []
    state = {"planted": planted, "bumps": [], "late_flags": [], "orphans": 0}
    order = list(range(n_kg))
    rng.shuffle(order)
    pending = [main_wg(J, n_qb, ctl, epoch, log, state) for J in order]
    pending.append(runner(n_qb, ctl, epoch, log))  # the runner that owns this (b, h)
    live, events, polls_in_a_row = [], 0, 0
    while pending or live:
        while pending and len(live) < resident:
            live.append(pending.pop(0))
        while state["bumps"] and rng.random() < 0.3:
            ctl.cnt[state["bumps"].pop(rng.randrange(len(state["bumps"])))] += 1
        if state["late_flags"] and rng.random() < 0.02:
            J, e = state["late_flags"].pop(0)
            ctl.orphan[J] = e
        k = rng.randrange(len(live))
        try:
            r = next(live[k])
        except StopIteration:
            live.pop(k)
            polls_in_a_row = 0
            continue
        events += 1
        polls_in_a_row = polls_in_a_row + 1 if r == "poll" and not state["bumps"] else 0
        assert polls_in_a_row < 200 * len(live) + 2000, \
            f"deadlock: n_qb={n_qb} resident={resident} seed={seed}"
        assert events < max_events, "no progress"
    for i in state["bumps"]:  # bumps still in flight land before the launch ends
        ctl.cnt[i] += 1
    for J, e in state["late_flags"]:
        ctl.orphan[J] = e
    return log, state["orphans"]


@pytest.mark.parametrize("n_qb", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("resident", [1, 2, 3, 4, 6])
def test_handover_schedules(n_qb, resident):
    n_kg = (n_qb + 1) // 2
    ctl = ControlBlock(n_qb, n_kg)
    ctl.orphan = [0xbeef] * n_kg  # stale flags of an unrelated launch
    for launch in range(60):
        epoch = launch + 1
        log, _ = run_launch(n_qb, resident, 1000 * n_qb + 10 * resident + launch, ctl, epoch)
        ran = sorted(J for J, _ in log)
        assert ran == list(range(n_kg)), f"items run {ran}, expected each of 0..{n_kg - 1} once"
        for J, complete in log:
            assert J == 0 or complete, f"item {J} ran before its counts were complete"
        assert ctl.cnt == [0] * n_qb
        assert ctl.done == 0


def test_orphans_happen_under_low_residency():
    """With few resident workgroups owners give up waiting and the runners
    take their items (the hand-over path is exercised, not just the waits)."""
    orphans = 0
    for seed in range(100):
        ctl = ControlBlock(8, 4)
        log, n = run_launch(8, 1 + seed % 3, seed, ctl, epoch=1)
        assert sorted(J for J, _ in log) == [0, 1, 2, 3]
        orphans += n
    assert orphans > 0


def test_model_catches_an_unbounded_owner_wait():
    """Planted mistake: owners wait without a bound. At low residency the
    model finds the deadlock."""
    found = False
    for seed in range(50):
        try:
            run_launch(8, 2, seed, ControlBlock(8, 4), epoch=1, planted="unbounded_owner")
        except AssertionError as e:
            assert "deadlock" in str(e)
            found = True
            break
    assert found


def test_model_catches_a_flag_seen_after_the_done_count():
    """Planted mistake: the orphan flag becomes visible after the done
    counter moved; a runner can then miss the item, which never runs."""
    lost = False
    for seed in range(300):
        log, n = run_launch(8, 1 + seed % 2, seed, ControlBlock(8, 4), epoch=1, planted="late_flag")
        if sorted(J for J, _ in log) != [0, 1, 2, 3]:
            lost = True
            break
    assert lost
