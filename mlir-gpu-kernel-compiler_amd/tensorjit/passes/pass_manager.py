"""Fixed-point pass driver; ``TENSORJIT_DUMP=1`` prints the IR after every
pass that changed it (ref ``tensorjit/passes/pass_manager.py:13-33``)."""
from __future__ import annotations

import os
import sys
from typing import Callable

from ..ir import Graph

Pass = Callable[[Graph], bool]


class PassManager:
    def __init__(self, passes: list[tuple[str, Pass]]):
        self.passes = passes
        self.dump = os.environ.get("TENSORJIT_DUMP", "0") == "1"

    def run(self, g: Graph, max_iters: int = 8) -> Graph:
        if self.dump:
            print(f"=== before passes ===\n{g}", file=sys.stderr)
        for it in range(max_iters):
            any_change = False
            for name, p in self.passes:
                if not p(g):
                    continue
                any_change = True
                g.toposort()
                if self.dump:
                    print(f"=== after {name} (iter {it}) ===\n{g}", file=sys.stderr)
            if not any_change:
                break
        g.toposort()
        return g
