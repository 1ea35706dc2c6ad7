"""The persistent decode kernel's item sub-queues hand out every work item
exactly once, whatever the grid (CPU check of the index rule the kernel uses,
csrc/paged_decode_mfma.hip): wavefront w starts with item w; sub-queue
q = w mod nq (nq = min(32, grid)) then serves first_queued(q) + nq * ticket,
first_queued(q) being the smallest index >= grid that is q modulo nq."""
import pytest

K_ITEM_QUEUES = 32  # kItemQueues in csrc/kernels.h


def served(grid: int, n_items: int):
    nq = min(K_ITEM_QUEUES, grid)
    seen = []
    for w in range(grid):
        if w < n_items:
            seen.append(w)
    for q in range(nq):
        first = q + nq * ((grid - q + nq - 1) // nq)
        i = first
        while i < n_items:
            seen.append(i)
            i += nq
    return seen


@pytest.mark.parametrize("grid", [1, 2, 7, 31, 32, 33, 40, 64, 100, 300, 2048])
@pytest.mark.parametrize("n_items", [1, 5, 32, 97, 1000, 6176])
def test_every_item_served_once(grid, n_items):
    got = sorted(served(grid, n_items))
    assert got == list(range(n_items))


def test_sub_queues_keep_list_order():
    """Within a sub-queue, tickets follow the (costliest-first) list order."""
    grid, n = 2048, 6176
    nq = min(K_ITEM_QUEUES, grid)
    for q in range(nq):
        first = q + nq * ((grid - q + nq - 1) // nq)
        seq = list(range(first, n, nq))
        assert seq == sorted(seq) and all(i % nq == q for i in seq)
