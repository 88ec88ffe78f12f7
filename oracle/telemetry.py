"""Route-reuse telemetry, CPU restatement (oracle, test infrastructure only).

Follows tarfa/engine/fused_int4.py:71-95: per layer a deque of the last 16
recorded expert sets; a decode step with experts ``el`` (sentinel dropped,
:165-167; nothing recorded when empty, :168) adds ``len(el)`` uses and, for each
window w in (1, 2, 4, 8, 16), ``|set(el) & union(last w sets)|`` reuses, then
appends ``set(el)``.  ``unique_layer_experts`` counts distinct (layer, expert).
"""
from collections import deque

WINDOWS = (1, 2, 4, 8, 16)


class RouteTelemetry:
    def __init__(self, layers):
        self.hist = {l: deque(maxlen=16) for l in range(layers)}
        self.per_layer = {l: {"decode_steps": 0, "expert_uses": 0, **{f"reuse_{w}": 0 for w in WINDOWS}}
                          for l in range(layers)}
        self.unique = set()

    def record(self, layer, ids, num_experts):
        el = [int(e) for e in ids if 0 <= int(e) < num_experts]
        if not el:
            return
        st = self.per_layer[layer]
        current = set(el)
        st["decode_steps"] += 1
        st["expert_uses"] += len(el)
        self.unique.update((layer, e) for e in current)
        previous = list(self.hist[layer])
        for w in WINDOWS:
            seen = set().union(*previous[-w:]) if previous else set()
            st[f"reuse_{w}"] += len(current & seen)
        self.hist[layer].append(current)

    def totals(self):
        out = {k: sum(st[k] for st in self.per_layer.values()) for k in self.per_layer[0]}
        out["unique_layer_experts"] = len(self.unique)
        return out
