"""CPU model of the single-launch GEMV completion protocol, explored over every
interleaving a small configuration allows.

The device code (gemv_kernel in strix-trellis_amd/csrc/gemv_kernel.hpp) runs,
per 128-column group and launch, S workgroups: splits 0..S-2 publish one
partial plane each and split S-1 (the finisher) polls for them.  Shared state
per column group: one epoch word, two plane sets, and the plan's sticky status.

  split s (s < S-1):  e = load(epoch)
                      store(planes[e & 1][s], partial)        } in either order
                      store(planes[(e & 1) ^ 1][s], EMPTY)    } (relaxed stores)
  finisher:           e = load(epoch)
                      poisoned (bit 31) or limit 0: give up at once
                      else load every word of planes[e & 1] until none is
                      EMPTY (at most `limit` rounds), then fold them in order
                      output = fold, or NaN on a give-up
                      give-up: status |= GAVE_UP, epoch = e | POISON
                      else:    epoch = (e + 1) & ~POISON

Launches of one plan are stream-ordered: launch k+1 starts after every
workgroup of launch k has ended.  Within a launch the adversary runs the
workgroups in any order, one memory access at a time -- a split may start
only after its finisher has given up (MI355X dispatches workgroups in grid
order only within one XCD).  Between launches the host may re-initialise the
state (strix_amd_plan_status with clear: status and epochs 0, planes EMPTY).

Safety property: a finisher that does not give up outputs exactly its own
launch's partials in split order.  The model checks it over every
interleaving (depth-first search with a visited set), and checks that the
previous protocol -- a give-up advanced the epoch and left the plan trusted --
violates it, i.e. that the model reaches the late-split case at all.
"""
import pytest

EMPTY = "EMPTY"
NAN = "NaN"
POISON = 1 << 31


def _value(launch, split):
    return f"L{launch}S{split}"


def explore(S, launches, limit, poison=True, resets=True):
    """Every reachable end state; returns (violations, finished runs, runs' output sequences).

    limit: poll rounds of every finisher, or a tuple with one per launch.

    A violation is (launch, output) where a non-NaN output is not the launch's
    own partials.  Workgroup states:
      split:    ("s", pc, e, pending)   pc 0: load epoch; 1: stores pending
      finisher: ("f", pc, e, idx, spin, got)
    """
    others = S - 1
    limits = tuple(limit) if isinstance(limit, (tuple, list)) else (limit,) * launches

    def fresh_launch():
        wgs = [("s", 0, None, None) for _ in range(others)]
        wgs.append(("f", 0, None, 0, 0, ()))
        return tuple(wgs)

    init = (0, (tuple([EMPTY] * others), tuple([EMPTY] * others)), 0, 0, fresh_launch(), ())
    seen = set()
    violations = []
    finished = 0
    runs = set()
    stack = [init]
    while stack:
        st = stack.pop()
        if st in seen:
            continue
        seen.add(st)
        epoch, planes, status, k, wgs, outs = st
        if all(w[0] == "done" for w in wgs):
            if k + 1 == launches:
                finished += 1
                runs.add(outs)
                continue
            nxt = [(epoch, planes, status, k + 1, fresh_launch(), outs)]
            if resets and status:
                nxt.append((0, (tuple([EMPTY] * others), tuple([EMPTY] * others)), 0, k + 1, fresh_launch(), outs))
            stack.extend(nxt)
            continue
        for i, w in enumerate(wgs):
            if w[0] == "done":
                continue
            if w[0] == "s":
                _, pc, e, pending = w
                if pc == 0:
                    new = ("s", 1, epoch, ("cur", "prev"))
                    stack.append((epoch, planes, status, k, wgs[:i] + (new,) + wgs[i + 1:], outs))
                    continue
                for which in pending:   # the two relaxed stores, in either order
                    cur = (e & 1)
                    target = cur if which == "cur" else cur ^ 1
                    word = _value(k, i) if which == "cur" else EMPTY
                    ps = [list(planes[0]), list(planes[1])]
                    ps[target][i] = word
                    rest = tuple(x for x in pending if x != which)
                    new = ("s", 1, e, rest) if rest else ("done",)
                    stack.append((epoch, (tuple(ps[0]), tuple(ps[1])), status, k, wgs[:i] + (new,) + wgs[i + 1:],
                                  outs))
                continue
            _, pc, e, idx, spin, got = w
            limit = limits[k]
            if pc == 0:   # load the epoch
                gave = limit == 0 or (poison and epoch & POISON)
                new = ("f", 2, epoch, 0, 0, NAN) if gave else ("f", 1, epoch, 0, 0, ())
                stack.append((epoch, planes, status, k, wgs[:i] + (new,) + wgs[i + 1:], outs))
            elif pc == 1:   # one plane word
                got = got + (planes[e & 1][idx],)
                if idx + 1 < others:
                    new = ("f", 1, e, idx + 1, spin, got)
                elif EMPTY not in got:
                    new = ("f", 2, e, 0, spin, got + (_value(k, others),))
                elif spin + 1 >= limit:
                    new = ("f", 2, e, 0, spin, NAN)
                else:
                    new = ("f", 1, e, 0, spin + 1, ())
                stack.append((epoch, planes, status, k, wgs[:i] + (new,) + wgs[i + 1:], outs))
            else:   # output, status and epoch
                gave = got == NAN
                if not gave and got != tuple(_value(k, s) for s in range(S)):
                    violations.append((k, got))
                if gave:
                    new_epoch = (e | POISON) if poison else (e + 1) & ~POISON
                    new_status = 1
                else:
                    new_epoch = (e + 1) & ~POISON
                    new_status = status
                stack.append((new_epoch, planes, new_status, k, wgs[:i] + (("done",),) + wgs[i + 1:],
                              outs + (got,)))
    return violations, finished, runs, len(seen)


@pytest.mark.parametrize("S,launches,limit", [(2, 3, 1), (2, 4, 2), (3, 3, 1), (3, 3, 2), (4, 3, 1)])
def test_poisoned_give_up_never_folds_a_stale_partial(S, launches, limit):
    violations, finished, runs, states = explore(S, launches, limit)
    print(f"S={S} launches={launches} limit={limit}: {states} states, {len(runs)} output sequences")
    assert finished > 0
    assert not violations, violations[:3]
    # Both outcomes occur: exact outputs, and give-ups (the adversary ran the
    # finisher's polls ahead of a split).
    outputs = {o for r in runs for o in r}
    assert NAN in outputs
    assert any(o != NAN for o in outputs)


@pytest.mark.parametrize("S,launches", [(2, 3), (3, 3)])
def test_exact_after_the_host_reinitialises(S, launches):
    # Launch 0 gives up at once (limit 0), and every split of it may still be
    # running or not yet started; the host clears; no later output folds a
    # stale partial, and a schedule exists in which launch 1 is exact.
    violations, _, runs, _ = explore(S, launches, limit=(0,) + (3,) * (launches - 1))
    assert not violations
    assert all(r[0] == NAN for r in runs)
    exact1 = tuple(_value(1, s) for s in range(S))
    assert any(r[1] == exact1 for r in runs)


def test_without_a_poison_a_late_split_is_folded():
    # The previous protocol: a give-up advanced the epoch and later finishers
    # trusted the planes.  A split of the given-up launch that starts after
    # the give-up reads the advanced epoch, publishes into the set the next
    # launch polls, and that launch's finisher folds the stale partial.
    violations, _, _, _ = explore(2, 2, limit=(0, 2), poison=False, resets=False)
    assert violations, "the model must reach a split that starts after its finisher gave up"
    k, got = violations[0]
    assert k == 1 and _value(0, 0) in got


def test_without_resets_a_poisoned_plan_stays_nan():
    # No host clear: after a give-up every later output of the run is NaN.
    violations, _, runs, _ = explore(3, 3, limit=1, resets=False)
    assert not violations
    for r in runs:
        if NAN in r:
            first = r.index(NAN)
            assert all(o == NAN for o in r[first:]), r
