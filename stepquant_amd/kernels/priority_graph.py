"""Decode graph with foreground priority (reference priority_graph.py:18-48).

The reference raises the priority of foreground kernel nodes on sm_80.  On
this platform every stream and graph node stays at default priority (mixed
priorities have hung these GPUs), so this is a plain graph that reports how
many of its kernel nodes would be foreground and background: ``(0, 0)``,
since nodes are not inspected.
"""
import torch


class PriorityDecodeGraph(torch.cuda.CUDAGraph):
    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self.priority_counts = (0, 0)
