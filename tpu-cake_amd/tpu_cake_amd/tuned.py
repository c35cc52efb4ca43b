"""Per-shape tuned knobs of the RPA kernel on gfx950.

The reference keys a table of Pallas block sizes on a simplified call shape and looks it up on
every call that leaves the block sizes unset (``get_tuned_block_sizes``,
``ecosystem/source/jax/ragged_paged_attention_tuned_block_sizes.py:1400-1486``: dtype names,
heads per block, head dim, page size, tokens and model length rounded up to powers of two).  The
HIP kernel has no block sizes -- its stream-K schedule balances work by itself -- so its table
holds the schedule knobs of ``rpa_options_t`` instead (``waves_per_cu``, ``prefill_tiles``,
``prefill_cost``), keyed on what moves them: the KV dtype, the GQA group G = Hq / Hkv, the page
size and the number of batched tokens, each rounded up to a power of two as upstream does.

The table is ``tuned_gfx950.json`` next to this module.  The knob search writes confirmed winners
into it (``tpu_cake_amd.search --promote``); a key that is not in it gets the library defaults.
"""

from __future__ import annotations

import functools
import json
import pathlib

DEVICE = "gfx950"
TABLE_PATH = pathlib.Path(__file__).with_name(f"tuned_{DEVICE}.json")
KNOBS = ("waves_per_cu", "prefill_tiles", "prefill_cost")
DEFAULTS = {"waves_per_cu": 0, "prefill_tiles": 0, "prefill_cost": 0.0}


def next_power_of_2(x: int) -> int:
    """Smallest power of two >= x (1 for x <= 1), as the reference's table key rounds."""
    x = int(x)
    return 1 if x <= 1 else 1 << (x - 1).bit_length()


def simplify_key(kv_dtype: str, group: int, page_size: int, num_tokens: int) -> str:
    """The table key of a call shape: ``"<kv dtype>/g<G>/p<page>/t<tokens>"`` with G, page size and
    tokens rounded up to powers of two."""
    if kv_dtype not in ("bf16", "fp8"):
        raise ValueError(f"kv_dtype must be 'bf16' or 'fp8', got {kv_dtype!r}")
    return f"{kv_dtype}/g{next_power_of_2(group)}/p{next_power_of_2(page_size)}/t{next_power_of_2(num_tokens)}"


def validate_entry(entry: dict) -> dict:
    """A table entry with every knob present and in range (ValueError otherwise)."""
    bad = set(entry) - set(KNOBS)
    if bad:
        raise ValueError(f"unknown knobs {sorted(bad)}")
    e = dict(DEFAULTS, **entry)
    if not (isinstance(e["waves_per_cu"], int) and 0 <= e["waves_per_cu"] <= 8):
        raise ValueError(f"waves_per_cu={e['waves_per_cu']!r} must be an int in [0, 8]")
    if isinstance(e["prefill_tiles"], bool):  # True: the library's choice; False: stream-K rows
        e["prefill_tiles"] = 0 if e["prefill_tiles"] else -1
    if e["prefill_tiles"] not in (-1, 0, 1, 2, 3):
        raise ValueError(f"prefill_tiles={e['prefill_tiles']!r} must be -1, 0, 1, 2 or 3 (or a bool)")
    if not (isinstance(e["prefill_cost"], (int, float)) and 0.0 <= float(e["prefill_cost"]) <= 64.0):
        raise ValueError(f"prefill_cost={e['prefill_cost']!r} must be in [0, 64]")
    e["prefill_cost"] = float(e["prefill_cost"])
    return e


@functools.lru_cache(maxsize=4)
def _load(path: str, mtime_ns: int) -> dict:
    data = json.loads(pathlib.Path(path).read_text())
    if data.get("device") != DEVICE:
        raise ValueError(f"{path}: table for device {data.get('device')!r}, expected {DEVICE!r}")
    return {k: validate_entry(v) for k, v in data.get("entries", {}).items()}


def table(path: pathlib.Path | None = None) -> dict:
    """key -> knob dict of the tuned table (empty when the file does not exist)."""
    path = pathlib.Path(path or TABLE_PATH)
    if not path.exists():
        return {}
    return _load(str(path), path.stat().st_mtime_ns)


def get_tuned_knobs(kv_dtype: str, group: int, page_size: int, num_tokens: int,
                    path: pathlib.Path | None = None) -> dict:
    """The knobs for a call shape: the table's entry for its key, else the library defaults."""
    return dict(table(path).get(simplify_key(kv_dtype, group, page_size, num_tokens), DEFAULTS))


def write_entry(key: str, knobs: dict, *, source: str, path: pathlib.Path | None = None) -> dict:
    """Insert or replace one entry (a confirmed search winner), recording where it came from."""
    path = pathlib.Path(path or TABLE_PATH)
    entry = validate_entry(knobs)
    data = json.loads(path.read_text()) if path.exists() else {"device": DEVICE, "entries": {}, "sources": {}}
    data.setdefault("entries", {})[key] = entry
    data.setdefault("sources", {})[key] = source
    path.write_text(json.dumps(data, indent=1, sort_keys=True) + "\n")
    _load.cache_clear()
    return entry
