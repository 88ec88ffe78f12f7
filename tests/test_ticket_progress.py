"""Forward progress of the fused decode's task graph under partial residency (CPU model).

The model restates the scheduling of tarfa_amd/csrc/decode_fused.hip: the task list order of
``decode_task`` (router rows R, then per slot j the gate/up tasks Gj, the down tasks D(j - 8)
after G j for j >= 8, the shared gate/up S after G(sh_after) -- right after R when sh_after
< 0, the int4 order --, the shared down SD after
G(sd_after), the remaining D last), its dependencies (S: none; SD: every S; Gj: every R;
Dj: every Gj; the last slot's D tasks, which combine, also every other slot's D task of the
same rows and the SD task of those rows), its queues (exact-bf16 mode: 128, task t in queue
t % 128, served by wave q % 4 of the blocks b of group q / 4, group(b) = (b % 8) * 4 + (b / 8) % 4;
int4 mode: 32, one group per XCD, group(b) = b % 8), and two
ticket rules: every ticket drawn from the queue's counter (what both modes of the kernel do),
or static tickets rank + users i (rank = b / 32), which the model keeps to show why they are
not used.

A step: every resident wave with no task draws its next ticket (or leaves when the ticket is
past its queue's tasks); a wave whose task's dependencies are all done finishes it.  Blocks
that are not resident do nothing; a block becomes resident at its arrival step when the GPU
has room (``capacity`` blocks), and leaves once its four waves have left.
"""
import pytest

KDOWNLAG, WAVES, GROUPS, GROUPS_INT4 = 8, 4, 32, 8


def group(b, groups=GROUPS):
    return b % 8 if groups == 8 else (b % 8) * 4 + (b // 8) % 4


def task_list(n_r, n_s, n_sd, n_g, n_d, k, sh_after, sd_after):
    """[(type, slot, idx)] in the order of decode_task (decode_fused.hip)."""
    out = [("R", 0, i) for i in range(n_r)]
    if sh_after < 0:
        out += [("S", 0, i) for i in range(n_s)]
    for j in range(k):
        out += [("G", j, i) for i in range(n_g)]
        if j >= KDOWNLAG:
            out += [("D", j - KDOWNLAG, i) for i in range(n_d)]
        if j == sh_after:
            out += [("S", 0, i) for i in range(n_s)]
        if j == sd_after:
            out += [("SD", k, i) for i in range(n_sd)]
    first = k - KDOWNLAG if k > KDOWNLAG else 0
    for j in range(first, k):
        out += [("D", j, i) for i in range(n_d)]
    return out


def dependencies(tasks, k):
    """Task index -> indices it waits on."""
    pos = {t: i for i, t in enumerate(tasks)}
    by = {}
    for i, (ty, slot, idx) in enumerate(tasks):
        by.setdefault((ty, slot), []).append(i)
    deps = []
    for ty, slot, idx in tasks:
        if ty in ("R", "S"):
            d = []
        elif ty == "SD":
            d = by[("S", 0)]
        elif ty == "G":
            d = by[("R", 0)]
        else:
            d = list(by[("G", slot)])
            if slot == k - 1:
                d += [pos[("D", j, idx)] for j in range(k - 1)]
                if ("SD", k, idx) in pos:
                    d.append(pos[("SD", k, idx)])
        deps.append(d)
    return deps


def simulate(tasks, deps, grid, dynamic, arrival, capacity, max_steps=5000, groups=GROUPS):
    """Run the model; returns (finished all, steps).  arrival[b] = step from which block b
    may become resident (None: never)."""
    n = len(tasks)
    done = [False] * n
    queues = groups * WAVES
    counters = [0] * queues
    first_block = {group(b, groups): b for b in reversed(range(groups))}
    users = [(grid - first_block[qq // WAVES] + groups - 1) // groups for qq in range(queues)]
    waves = {}          # (block, wave) -> {"ticket_i": i, "task": t or None, "left": bool}
    resident, finished_blocks = set(), set()
    for step in range(max_steps):
        # arrivals, in block order, while there is room
        for b in range(grid):
            if b in resident or b in finished_blocks or arrival[b] is None or arrival[b] > step:
                continue
            if len(resident) >= capacity:
                break
            resident.add(b)
            for w in range(WAVES):
                waves[(b, w)] = {"i": 0, "task": None, "left": False}
        progressed = False
        for (b, w), st in waves.items():
            if b not in resident or st["left"]:
                continue
            q = group(b, groups) * WAVES + w
            if st["task"] is None:
                if dynamic:
                    ticket = counters[q]
                    counters[q] += 1
                else:
                    ticket = b // groups + users[q] * st["i"]
                st["i"] += 1
                t = q + queues * ticket
                if t >= n:
                    st["left"] = True
                    progressed = True
                    continue
                st["task"] = t
                progressed = True
            t = st["task"]
            if all(done[d] for d in deps[t]):
                done[t] = True
                st["task"] = None
                progressed = True
        for b in list(resident):
            if all(waves[(b, w)]["left"] for w in range(WAVES)):
                resident.discard(b)
                finished_blocks.add(b)
                progressed = True
        if all(done):
            return True, step
        pending_arrivals = any(arrival[b] is not None and arrival[b] > step and b not in finished_blocks
                               for b in range(grid))
        if not progressed and not pending_arrivals:
            return False, step
    return all(done), max_steps


FULL = dict(n_r=65, n_s=512, n_sd=320, n_g=512, n_d=320, k=8, sh_after=1, sd_after=7)
# Int4 mode at the same layer: 4 row pairs per gate/up task, 16 rows per down task, S first.
FULL_INT4 = dict(n_r=65, n_s=256, n_sd=320, n_g=256, n_d=160, k=8, sh_after=-1, sd_after=7)


def _graph(shape=FULL):
    tasks = task_list(**shape)
    deps = dependencies(tasks, shape["k"])
    return tasks, deps


def test_int4_order_completes_with_drawn_tickets_and_partial_residency():
    tasks, deps = _graph(FULL_INT4)
    assert len(tasks) == 65 + 256 + 320 + 8 * (256 + 160)
    assert tasks[65] == ("S", 0, 0) and tasks[65 + 256] == ("G", 0, 0)
    for i, d in enumerate(deps):
        assert all(j < i for j in d), (i, tasks[i])
    g = GROUPS_INT4
    assert simulate(tasks, deps, 512, True, [0] * 512, capacity=512, groups=g)[0]
    # One block per XCD (blocks 0..7), room for 40 blocks, late blocks.
    assert simulate(tasks, deps, 512, True, [0 if b < g else None for b in range(512)], capacity=512, groups=g)[0]
    assert simulate(tasks, deps, 512, True, [0] * 512, capacity=40, groups=g)[0]
    arrival = [0 if b % 7 == 0 or b < g else 3 + (b * 37) % 50 for b in range(512)]
    assert simulate(tasks, deps, 512, True, arrival, capacity=96, groups=g)[0]
    # Static tickets would not: one block never resident stalls the int4 order too.
    arrival = [None if b == 9 else 0 for b in range(512)]
    assert not simulate(tasks, deps, 512, False, arrival, capacity=512, groups=g)[0]


def test_every_dependency_points_to_a_smaller_task():
    tasks, deps = _graph()
    assert len(tasks) == 65 + 512 + 320 + 8 * (512 + 320)
    for i, d in enumerate(deps):
        assert all(j < i for j in d), (i, tasks[i])


@pytest.mark.parametrize("dynamic", [True, False])
def test_whole_grid_resident_completes(dynamic):
    tasks, deps = _graph()
    ok, _ = simulate(tasks, deps, 512, dynamic, [0] * 512, capacity=512)
    assert ok


def test_dynamic_tickets_complete_with_blocks_missing_or_late():
    tasks, deps = _graph()
    # Only one block per group ever resident (blocks 0..31): every queue keeps one server.
    arrival = [0 if b < GROUPS else None for b in range(512)]
    assert simulate(tasks, deps, 512, True, arrival, capacity=512)[0]
    # Room for 40 blocks: the rest arrive as earlier blocks leave.
    assert simulate(tasks, deps, 512, True, [0] * 512, capacity=40)[0]
    # Late blocks of every XCD, in a scrambled order.
    arrival = [0 if b % 7 == 0 or b < GROUPS else 3 + (b * 37) % 50 for b in range(512)]
    assert simulate(tasks, deps, 512, True, arrival, capacity=96)[0]


def test_static_tickets_stall_when_a_block_is_missing():
    tasks, deps = _graph()
    # Block 9 (group 5, rank 0) never resident: its static first tickets (router tasks among
    # them) are never run, and every gate/up task waits on the routing.
    arrival = [None if b == 9 else 0 for b in range(512)]
    assert not simulate(tasks, deps, 512, False, arrival, capacity=512)[0]
    assert simulate(tasks, deps, 512, True, arrival, capacity=512)[0]
    # Room for fewer blocks than the grid: resident waves spin on tasks whose static owners
    # cannot arrive until they leave.
    assert not simulate(tasks, deps, 512, False, [0] * 512, capacity=40)[0]


def test_dynamic_tickets_need_one_server_per_queue():
    tasks, deps = _graph()
    # No block ever on XCD 3: queues 48..63 have no server, and their tasks never run.
    arrival = [None if b % 8 == 3 else 0 for b in range(512)]
    assert not simulate(tasks, deps, 512, True, arrival, capacity=512)[0]
