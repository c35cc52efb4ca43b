"""The reference's canonical schedule text for the v1 Inkling workload (``inkling-rpa``).

The reference renders a workload's schedule as the generic-form MLIR text of an xDSL module of its
``tpu_schedule`` dialect (``canonical_module_text``, ``src/tpu_cake/frontend.py:633-638``) and
pins an experiment to the sha256 of that text (``schedule_sha256``).  For ``inkling-rpa`` the
module is built by ``inkling_rpa_schedule`` (``src/tpu_cake/workloads/inkling_rpa.py:87-143``):
a ``tpu_schedule.kernel`` whose block arguments are the seven HBM buffers, three VMEM
allocations, three semaphores, DMAs in and out around one ``tpu_schedule.ragged_paged_attention``
op, and a yield; the checked-in rendering is ``examples/inkling-rpa.mlir``.

This build does not carry the xDSL IR (out of scope: it targets TPU7x); this module writes that
one text format directly, so ``render-workload inkling-rpa`` still prints the reference's schedule
and ``experiment inkling-rpa`` still pins its sha256.
"""

from __future__ import annotations

import dataclasses


@dataclasses.dataclass(frozen=True)
class Buffer:
    """``!tpu_schedule.buffer``: memref shape and element type, logical dim names, memory space,
    ownership and lifetime (row-major layout, no sharding)."""
    shape: tuple
    names: str
    dtype: str
    memory: str = "hbm"
    ownership: str = "external"
    lifetime: tuple = (0, 4)

    def type(self) -> str:
        dims = "x".join(str(d) for d in self.shape) + "x" + self.dtype
        names = ", ".join(f'"{n}"' for n in self.names.split())
        shard = ", ".join('""' for _ in self.shape)
        layout = ", ".join(f"#builtin.int<{i}>" for i in range(len(self.shape)))
        a, b = self.lifetime
        return (f"!tpu_schedule.buffer<memref<{dims}>, #tpu_schedule.shape<[{names}]>, "
                f"#tpu_schedule<memory_space {self.memory}>, #tpu_schedule.sharding<[{shard}]>, "
                f"#tpu_schedule.layout<[{layout}]>, #tpu_schedule<ownership {self.ownership}>, "
                f"#tpu_schedule.lifetime<#builtin.int<{a}>, #builtin.int<{b}>>>")


SEMAPHORE = "!tpu_schedule.semaphore"
DMA_TOKEN = "!tpu_schedule.dma_token"


def _int(v: int) -> str:
    return f"#builtin.int<{v}>"


class KernelText:
    """Builds the generic-form text of one ``tpu_schedule.kernel`` module: SSA values are numbered
    in definition order (block arguments first), one op per line."""

    def __init__(self, name: str, target: str, inputs, *, vmem_capacity_bytes: int, smem_capacity_bytes: int):
        self.header = (f'"tpu_schedule.kernel"() <{{sym_name = "{name}", target = "{target}", '
                       f"vmem_capacity_bytes = {_int(vmem_capacity_bytes)}, "
                       f"smem_capacity_bytes = {_int(smem_capacity_bytes)}}}> ({{")
        self.types: list[str] = [b.type() for b in inputs]
        self.args = len(self.types)
        self.lines: list[str] = []

    def _value(self, typ: str) -> int:
        self.types.append(typ)
        return len(self.types) - 1

    def alloc(self, buf: Buffer, role: str) -> int:
        v = self._value(buf.type())
        self.lines.append(f'%{v} = "tpu_schedule.alloc"() <{{role = "{role}"}}> : () -> {buf.type()}')
        return v

    def semaphore(self) -> int:
        v = self._value(SEMAPHORE)
        self.lines.append(f'%{v} = "tpu_schedule.semaphore_alloc"() : () -> {SEMAPHORE}')
        return v

    def _operands(self, vals) -> tuple[str, str]:
        return ", ".join(f"%{v}" for v in vals), ", ".join(self.types[v] for v in vals)

    def dma_start(self, src: int, dst: int, sem: int, *, stage: int) -> int:
        ops, tys = self._operands((src, dst, sem))
        v = self._value(DMA_TOKEN)
        self.lines.append(f'%{v} = "tpu_schedule.dma_start"({ops}) <{{stage = {_int(stage)}}}> : ({tys}) -> {DMA_TOKEN}')
        return v

    def dma_wait(self, token: int, *, stage: int) -> None:
        self.lines.append(f'"tpu_schedule.dma_wait"(%{token}) <{{stage = {_int(stage)}}}> : ({DMA_TOKEN}) -> ()')

    def op(self, name: str, vals, **attrs: int) -> None:
        ops, tys = self._operands(vals)
        at = ", ".join(f"{k} = {_int(v)}" for k, v in attrs.items())
        self.lines.append(f'"tpu_schedule.{name}"({ops}) <{{{at}}}> : ({tys}) -> ()')

    def text(self) -> str:
        args = ", ".join(f"%{i}: {t}" for i, t in enumerate(self.types[: self.args]))
        body = [f"    {line}" for line in self.lines + ['"tpu_schedule.yield"() : () -> ()']]
        return "\n".join(['"builtin.module"() ({', "  " + self.header, f"  ^bb0({args}):", *body,
                          "  }) : () -> ()", "}) : () -> ()"]) + "\n"


def inkling_rpa_schedule_text() -> str:
    """The reference's ``inkling-rpa`` schedule (inkling_rpa.py:87-143) as its canonical text."""
    bf16, i32 = "bf16", "i32"
    inputs = (
        Buffer((4, 4, 32), "B H D", bf16),
        Buffer((32, 16, 4, 32), "P S H D", bf16),
        Buffer((32, 16, 4, 32), "P S H D", bf16),
        Buffer((4, 8), "B MP", i32),
        Buffer((4,), "B", i32),
        Buffer((4, 128), "H L", bf16),
        Buffer((4, 4, 32), "B H D", bf16),
    )
    k = KernelText("inkling_rpa_decode", "tpu7x", inputs, vmem_capacity_bytes=2 << 20, smem_capacity_bytes=1 << 16)
    local = dict(memory="vmem", ownership="kernel")
    query = k.alloc(Buffer((4, 4, 32), "B H D", bf16, lifetime=(0, 2), **local), "query_tile")
    bias = k.alloc(Buffer((4, 128), "H L", bf16, lifetime=(0, 2), **local), "relative_bias")
    output = k.alloc(Buffer((4, 4, 32), "B H D", bf16, lifetime=(2, 4), **local), "attention_output")
    q_sem, b_sem, o_sem = k.semaphore(), k.semaphore(), k.semaphore()
    q_dma = k.dma_start(0, query, q_sem, stage=0)
    b_dma = k.dma_start(5, bias, b_sem, stage=0)
    k.dma_wait(q_dma, stage=1)
    k.dma_wait(b_dma, stage=1)
    k.op("ragged_paged_attention", (query, 1, 2, 3, 4, bias, output), stage=2, query_block_size=1, kv_block_size=8)
    o_dma = k.dma_start(output, 6, o_sem, stage=3)
    k.dma_wait(o_dma, stage=4)
    return k.text()
