"""The host slot pool (kvm_slot_pool) against the reference adapter's free list
(reset_slots / alloc_slot / free_slot, llama-memory-kvmem.cpp:1018-1024,
1720-1741), restated as a Python list: pushed n-1 .. 0, allocation pops the
back, freeing pushes."""
import numpy as np

from kvmem_amd import api


class _RefPool:
    def __init__(self, n):
        self.n = n
        self.reset()

    def reset(self):
        self.free = list(range(self.n - 1, -1, -1))

    def alloc(self):
        return self.free.pop() if self.free else -1

    def release(self, slot):
        if slot >= 0:
            self.free.append(slot)


def test_first_allocations_are_in_slot_order():
    p = api.SlotPool(6)
    assert [p.alloc() for _ in range(7)] == [0, 1, 2, 3, 4, 5, -1]


def test_random_sequences_match_the_reference_free_list():
    rng = np.random.default_rng(8)
    for n in (1, 5, 36, 256):
        p, r = api.SlotPool(n), _RefPool(n)
        held = []
        for _ in range(600):
            op = rng.random()
            if op < 0.5:
                a, b = p.alloc(), r.alloc()
                assert a == b
                if a >= 0:
                    held.append(a)
            elif op < 0.95 and held:
                s = held.pop(int(rng.integers(0, len(held))))
                p.free(s)
                r.release(s)
            elif op < 0.97:
                p.free(-1)
                r.release(-1)
            else:
                p.reset()
                r.reset()
                held = []
        assert [p.alloc() for _ in range(n + 1)] == [r.alloc() for _ in range(n + 1)]
