"""A decode session: one decoder step program, gated, planned, lowered and
resident on one GPU, stepped token by token.

The engine writes the program (``program.decoder``), the gate checks it, the
planner cuts it into steps, the lowering picks a kernel per step, and the
engine keeps weights and KV caches in HBM across steps.  ``graph()`` captures a
whole step — and the device-side advance of its token and position — so a
token costs one graph replay.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional

import numpy as np

from . import kernels as K
from . import runtime
from .engine import Engine
from .lower import lower_plan
from .program.check import check_program
from .program.decoder import DecoderDims, decoder_step
from .program.graph import SCache, SInput, SWeight
from .program.plan import PlanOptions, plan


@dataclass
class DecodeSession:
    device: runtime.Device
    kernels: K.Kernels
    dims: DecoderDims
    options: PlanOptions
    embed: bool = True
    layers: Optional[int] = None
    fuse: bool = True
    tuned: bool = False  # shape the GEMV steps as the committed selections pick
    paging: Optional[tuple] = None  # (block size, pool blocks): the caches as paged pools
    choose: Optional[Callable] = None  # the GEMV steps' (rows a block, threadgroups a CU), as lower_plan takes

    def __post_init__(self):
        self.program = decoder_step(self.dims, embed=self.embed, layers=self.layers, paging=self.paging)
        self.checked = check_program(self.program)
        self.plan = plan(self.options, self.checked)
        choose = self.choose
        if self.tuned and choose is None:
            from .tuning import committed_chooser
            choose = committed_chooser(self.device.info.compute_units)
        self.lowered = lower_plan(self.checked, self.plan, fuse=self.fuse,
                                  compute_units=self.device.info.compute_units if choose else 256,
                                  choose=choose)
        self.engine = Engine(self.device, self.kernels, self.lowered)

    # Synthetic state ------------------------------------------------------------

    def init_synthetic(self, seed: int = 2026, std: float = 0.02, cache_seed: int = 2027) -> None:
        """Weights std * N(0, 1) (norm gains 1), caches N(0, 1), as the
        configurations have them; all generated on the device."""
        for i, src in enumerate(self.program.sources):
            name = f"weight:{src.name}"
            if isinstance(src.kind, SWeight) and name in self.lowered.buffers:
                if len(src.kind.dims) == 1:
                    self.engine.write(name, np.ones(src.kind.dims[0], np.float32))
                else:
                    self.engine.init_normal(name, seed + 7919 * i, std)
            if f"widen:{src.name}" in self.lowered.buffers:
                self.engine.write(f"widen:{src.name}", np.ones(int(np.prod(src.kind.dims)), np.float32))
            if isinstance(src.kind, SCache):
                self.engine.init_normal(f"cache:{src.name}", cache_seed + 7919 * i, 1.0)
            if isinstance(src.kind, SInput):
                self.engine.init_normal(f"value:{src.name}", cache_seed + 104729 * i, std)
        self.device.sync()

    def set_position(self, position: int, slot: int = 0, token: Optional[int] = None,
                     table: Optional[np.ndarray] = None) -> None:
        """The row's position and ring slot, or with paged pools its block
        table (the context's positions in blocks)."""
        self.engine.set_ints("position", [position], self.dims.context)
        if self.paging is None:
            self.engine.set_ints("slot", [slot], self.dims.slots)
        else:
            block_size, pool_blocks = self.paging
            if table is None or len(table) != self.dims.context // block_size:
                raise ValueError(f"a block table of {self.dims.context // block_size} blocks")
            self.engine.set_ints("blocks", table, pool_blocks)
        if self.embed and token is not None:
            self.engine.set_ints("tokens", [token], self.dims.vocab)

    # Running ------------------------------------------------------------------

    def step(self) -> None:
        self.engine.enqueue()

    def graph(self, advance_position: bool = True) -> runtime.Graph:
        advance = None
        if self.embed:
            advance = dict(token_out="value:token", token_in="ints:tokens", position="ints:position",
                           context=self.dims.context, step=1 if advance_position else 0)
        return self.engine.capture(advance)

    def token(self) -> int:
        return int(self.engine.read("value:token")[0])

    def logits(self) -> np.ndarray:
        return self.engine.read("value:logits")

    def close(self) -> None:
        self.engine.close()
