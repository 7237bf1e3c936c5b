"""TEST INFRASTRUCTURE ONLY: the reference expert cache's LRU bookkeeping
(usaf/moe_loader.py:130-181 get_expert_weights) restated for arbitrary keys,
the checker of usaf_amd's per-expert slot cache.

A hit moves the key to the most recent end (:145-146); a miss first evicts
least recently used keys while the cache is full (:166-167), then inserts the
key at the most recent end (:177).  Resident modules (:153-164) and the
prefetch hand-over (:169-173) do not change this order and are left out.
"""
from __future__ import annotations

from collections import OrderedDict


class LRUModel:
    def __init__(self, capacity: int) -> None:
        self.capacity = capacity
        self.order: "OrderedDict[object, None]" = OrderedDict()

    def access(self, key):
        """(hit, evicted keys) of one access."""
        if key in self.order:
            self.order.move_to_end(key)
            return True, []
        evicted = []
        while len(self.order) >= self.capacity:
            evicted.append(self.order.popitem(last=False)[0])
        self.order[key] = None
        return False, evicted

    def keys(self):
        return list(self.order.keys())
