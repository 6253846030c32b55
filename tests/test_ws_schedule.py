"""Host-level check of the wave-specialised moment scan's per-iteration schedule (csrc/moments_ws.hip,
ws_body): which LDS buffer, handoff copy and register every step of the update and query waves writes
and reads, iteration by iteration, with one barrier at the end of each iteration.

The model follows the kernel's program order for each role:
  update waves, iteration c: [staging of chunk c + 1's keys / values and chunk c's queries, the loads of
    the next slot], the reduction of the query waves' partials of chunk c - 2, the update of chunk c,
    and after the last chunk of a block the state handoff (global memory, copy by block parity when a
    block is 2 chunks, one copy otherwise) and the block's denominators (LDS, by block parity);
  query waves, iteration c: the products of chunk c - 1 against their frozen state, their partials of
    chunk c - 1, [their share of the staging where all 512 threads stage], and at the first chunk of a
    block the reload of the new block's state from the handoff and of its denominators.
Accesses of the two roles to one location in one iteration are unordered (a race when one writes).
The handoff reload is a global load: it may still be in flight after the barrier and lands before the
query waves' first use of the state one iteration later, so a write to its copy before that use is a
race too.  Every read must see the version the algorithm needs (the keys of chunk c, the state before
the block of the rows it answers, ...).  The shipped order passes for every block length; the reference
semantics it preserves are fast_article_attention.py:217-259 (rows see the keys before their block).

Two other orders are checked for what they would do: the query waves staging before their products with
the reload after them (hazard-free, like the shipped order) and the whole staging step, reload
included, before the products (rows of a block's last chunk answered from the next block's state)."""

import pytest

SHIPPED, STAGE_FIRST, RELOAD_FIRST = "shipped", "stage_first", "reload_first"


class Race(AssertionError):
    pass


def simulate(cpb: int, nch: int, query_stages: bool, order: str, copies: int = 0) -> None:
    """Runs the schedule of one workgroup over nch chunks with query blocks of cpb chunks; raises Race
    or AssertionError on the first hazard or wrong version.  copies: handoff copies (0: the kernel's
    rule, one copy for cpb >= 3 and two alternating by block parity for cpb = 2)."""
    if copies == 0:
        copies = 1 if cpb >= 3 else 2  # the kernel's hmask
    mem = {}  # location -> version tag
    block = lambda c: c // cpb  # noqa: E731
    for p in (0, 1):
        mem[("den", p)] = ("D", 0)  # zeroed: the state before block 0 is empty
    mem[("kv", 0)] = ("K", 0)  # the prologue stages chunk 0's keys and values before the first barrier
    sh = ("S", 0)  # the query waves' frozen state (registers), block 0's state is zero
    dh = ("D", 0)
    pending = None  # (copy, expected tag, iteration issued): a handoff reload still in flight
    for c in range(nch + 1):
        acc = {"upd": [], "qry": []}  # (kind, location) of this iteration, for the cross-role check

        def write(role, loc, tag):
            acc[role].append(("w", loc))
            mem[loc] = tag

        def read(role, loc, want, what):
            acc[role].append(("r", loc))
            got = mem.get(loc)
            if got != want:
                raise AssertionError(f"cpb {cpb} iteration {c}: {what} read {got} from {loc}, needs {want}")

        def stage(role):
            # where both roles stage, each writes its own units of the chunk (disjoint parts: "s")
            if c + 1 < nch:
                write(role, ("kv", (c + 1) & 1), ("K", c + 1))
                acc[role][-1] = ("s", ("kv", (c + 1) & 1))
            if c < nch:
                write(role, ("q", c & 1), ("Q", c))
                acc[role][-1] = ("s", ("q", c & 1))

        # ---- update waves ----
        stage("upd")
        if c >= 2:
            read("upd", ("red", c & 1), ("P", c - 2), "reduction")
        if c < nch:
            read("upd", ("kv", c & 1), ("K", c), "update")
            if (c + 1) % cpb == 0 and c + 1 < nch:
                b = (c + 1) // cpb
                write("upd", ("hand", b % 2 if copies == 2 else 0), ("S", b))
                write("upd", ("den", b & 1), ("D", b))

        # ---- query waves ----
        def reload():
            nonlocal pending, dh
            if c >= 1 and c % cpb == 0 and c < nch:
                b = c // cpb
                copy = b % 2 if copies == 2 else 0
                acc["qry"].append(("r", ("hand", copy)))
                pending = (copy, mem.get(("hand", copy)), ("S", b), c)
                read("qry", ("den", b & 1), ("D", b), "denominator reload")
                dh = ("D", b)

        def products():
            nonlocal sh, pending
            if c >= 1:
                if pending is not None and pending[3] < c:  # the reload lands before its first use
                    copy, got, want, _ = pending
                    if mem.get(("hand", copy)) != got:
                        raise Race(f"cpb {cpb} iteration {c}: handoff copy {copy} rewritten before the reload landed")
                    if got != want:
                        raise AssertionError(f"cpb {cpb}: reload got {got}, needs {want}")
                    sh, pending = got, None
                need = ("S", block(c - 1))
                read("qry", ("q", (c - 1) & 1), ("Q", c - 1), "query products")
                if sh != need or dh != ("D", block(c - 1)):
                    raise AssertionError(f"cpb {cpb} iteration {c}: chunk {c - 1} answered with {sh} / {dh}, "
                                         f"needs {need}")
                write("qry", ("red", (c - 1) & 1), ("P", c - 1))

        if order == SHIPPED:
            products()
            if query_stages:
                stage("qry")
            reload()
        elif order == STAGE_FIRST:
            if query_stages:
                stage("qry")
            products()
            reload()
        else:
            if query_stages:
                stage("qry")
            reload()
            products()

        # ---- cross-role hazards within the iteration (the barrier orders everything else) ----
        for kind_u, loc_u in acc["upd"]:
            for kind_q, loc_q in acc["qry"]:
                if loc_u == loc_q and (kind_u, kind_q) != ("s", "s") and (kind_u, kind_q) != ("r", "r"):
                    raise Race(f"cpb {cpb} iteration {c}: update and query waves both access {loc_u}")
        # a reload in flight across the barrier: its copy must not be written until it lands
        if pending is not None and pending[3] < c and mem.get(("hand", pending[0])) != pending[1]:
            raise Race(f"cpb {cpb} iteration {c}: handoff copy {pending[0]} rewritten under an in-flight reload")


@pytest.mark.parametrize("cpb", [2, 3, 4, 5, 8])
@pytest.mark.parametrize("query_stages", [False, True])
def test_shipped_schedule_is_hazard_free(cpb, query_stages):
    for nch in range(1, 6 * cpb + 3):
        simulate(cpb, nch, query_stages, SHIPPED)


@pytest.mark.parametrize("cpb", [2, 3, 4])
def test_query_staging_first_is_hazard_free_too(cpb):
    """Staging before the products with the reload after them: the order described for the dropped
    variant has no hazard in this model either."""
    for nch in range(1, 6 * cpb + 3):
        simulate(cpb, nch, True, STAGE_FIRST)


@pytest.mark.parametrize("cpb", [2, 3, 4])
def test_reload_before_products_answers_from_the_next_block(cpb):
    with pytest.raises(AssertionError, match="answered with"):
        simulate(cpb, 4 * cpb, True, RELOAD_FIRST)


def test_one_handoff_copy_at_two_chunks_per_block_races():
    """Why two copies at cpb = 2: with one, the update waves rewrite the copy in the iteration in which
    the query waves' reload of it lands (a planted mistake in the model, not in the kernel)."""
    with pytest.raises(Race):
        simulate(2, 8, False, SHIPPED, copies=1)
    simulate(3, 12, False, SHIPPED, copies=1)
