"""Write golden vectors from the reference implementation (run in the build container only).

Usage: python tests/golden/make_vectors.py [/path/to/reference]

Imports the reference package from <reference>/src (default /root/reference)
to record the outputs of the functions that the oracle's own checks do not
pin completely:
  - codec.code_lengths / Code / encode: the exact record bytes and LUT
    (codec.py:61-193) depend on heap tie-breaking and the refill reorder;
  - ExpertTable.seed / plan_chunks / acquire sequences (table.py:75-247):
    exact arrays on random multi-step traces.
Only inputs and outputs are saved (npz, no pickles); the reference never
leaves this container. Working steps use routing whose referenced experts all
have distinct counts, so torch.topk's unspecified tie order cannot matter.
"""

import os
import random
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _load_reference(root: str):
    sys.path.insert(0, os.path.join(root, "src"))
    from vllm_expert_pager import codec, table  # noqa: E402

    return codec, table


EXP_P = [0.0] * 4 + [0.001, 0.002, 0.004, 0.008, 0.016, 0.032, 0.064, 0.125, 0.228, 0.315, 0.188, 0.015]


def _rows(seed: int, n: int, p) -> np.ndarray:
    rng = np.random.default_rng(seed)
    p = np.asarray(p, np.float64)
    exp = rng.choice(16, size=n, p=p / p.sum()).astype(np.uint8)
    sm = rng.integers(0, 256, size=n, dtype=np.uint8) & 0x87
    return sm | (exp << 3)


def _fp8_row(seed: int, rows: int, cols: int) -> np.ndarray:
    """N(0, 0.02) weights quantised to e4m3 with 128x128 block scales."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn((rows, cols), generator=g) * 0.02
    q = torch.empty((rows, cols), dtype=torch.float8_e4m3fn)
    for r0 in range(0, rows, 128):
        for c0 in range(0, cols, 128):
            blk = w[r0 : r0 + 128, c0 : c0 + 128]
            s = blk.abs().max().clamp(min=1e-12) / 448.0
            q[r0 : r0 + 128, c0 : c0 + 128] = (blk / s).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).numpy().reshape(-1).copy()


def codec_vectors(codec) -> dict:
    out = {}
    cases = [
        ("realistic", _rows(0, 2 * 64 * 32, EXP_P), 64, 1.25),
        ("uniform", _rows(1, 2 * 64 * 32, [1.0] * 16), 64, 1.25),
        ("geometric", _rows(2, 2 * 64 * 32, [2.0**k for k in range(16)]), 64, 1.25),
        ("constant", np.full(2 * 64 * 32, 13 << 3, np.uint8), 64, 1.25),
        ("fp8_one_group", _fp8_row(3, 128, 128), 512, 1.0),
        ("fp8_two_groups", _fp8_row(4, 128, 256), 512, 0.95),
    ]
    names = []
    for name, raw, chunk, ratio in cases:
        pitch = codec.pitch_of(raw.size, ratio, 4096)
        rec, lut = codec.encode(torch.from_numpy(raw.copy()), pitch, chunk)
        out[f"{name}_raw"] = raw
        out[f"{name}_chunk"] = np.array(chunk)
        out[f"{name}_pitch"] = np.array(pitch)
        out[f"{name}_record"] = rec.numpy()
        out[f"{name}_lut"] = lut.numpy()
        names.append(name)
    out["cases"] = np.array(names)
    # code_lengths / Code on assorted histograms, including ones that need
    # the length limit and ones full of ties.
    hists = [
        [2**k for k in range(16)],
        [1] * 16,
        [0] * 16,
        [0] * 13 + [5, 0, 0],
        [3, 3, 3, 3, 7, 7, 7, 7, 100, 100, 1, 1, 0, 0, 9, 9],
        [int(x * 100000) for x in EXP_P],
        [1 << 40] + [1] * 15,
    ]
    rng = random.Random(5)
    for _ in range(24):
        hists.append([rng.choice([0, 1, 2, rng.randrange(1, 1000), rng.randrange(1, 10**7)]) for _ in range(16)])
    out["hists"] = np.array(hists, np.int64)
    out["lengths"] = np.array([codec.code_lengths(h) for h in hists], np.int64)
    out["codes"] = np.array([codec.Code(h).codes for h in hists], np.int64)
    out["luts"] = np.array([codec.Code(h).lut for h in hists], np.int64)
    return out


def _distinct_count_ids(rng: random.Random, E: int, k: int) -> list[int]:
    experts = rng.sample(range(E), k)
    ids = []
    for i, e in enumerate(experts):
        ids += [e] * (k - i)
    rng.shuffle(ids)
    return ids


def table_vectors(table, E, S, R, W, L, layer, steps, seed) -> dict:
    ExpertTable = table.ExpertTable
    cpu = torch.device("cpu")
    rng = random.Random(seed)
    vram, ram = ExpertTable(E, S, cpu), ExpertTable(E, R, cpu)
    ram.slot_of[:R] = ram.experts[:R]
    ram.expert_in[:R] = ram.experts[:R]
    out = {"E": np.array(E), "S": np.array(S), "R": np.array(R), "W": np.array(W), "L": np.array(L),
           "layer": np.array(layer), "steps": np.array(steps)}

    def state(prefix, t):
        out[prefix + "slot_of"] = t.slot_of[: t.num_experts].numpy().copy()
        out[prefix + "expert_in"] = t.expert_in[: t.num_slots].numpy().copy()
        out[prefix + "last_used"] = t.last_used[: t.num_slots].numpy().copy()
        out[prefix + "counters"] = np.array([int(t.step), int(t.hits), int(t.misses)])

    for i in range(steps):
        p = f"s{i}_"
        if rng.random() < 0.5:
            k = rng.randint(1, S)
            ids = [rng.randrange(E) for _ in range(k)]
            if rng.random() < 0.2:
                ids[rng.randrange(k)] = -1
            t_ids = torch.tensor([ids], dtype=torch.int32)
            emap, slot, todo = vram.acquire(t_ids)
            _, rslot, rtodo = ram.acquire(t_ids)
            out[p + "kind"] = np.array(0)
            out[p + "ids"] = np.array(ids, np.int64)
            out[p + "emap"] = emap.numpy().copy()
            out[p + "slot"] = slot.numpy().copy()
            out[p + "todo"] = todo.numpy().copy()
            out[p + "rslot"] = rslot.numpy().copy()
            out[p + "rtodo"] = rtodo.numpy().copy()
        else:
            k = rng.randint(S + 1, min(E, S + 2 * W + 4))
            ids = _distinct_count_ids(rng, E, k)
            t_ids = torch.tensor([ids], dtype=torch.int32)
            need = ram.need_mask(t_ids)
            cached_row = vram.slot_of[:E].clone()
            before = ram.slot_of[:E].clone()
            if t_ids.numel() <= R:
                ram.acquire(t_ids)
                out[p + "kind"] = np.array(1)
            else:
                ram.seed(vram, t_ids, need)
                out[p + "kind"] = np.array(2)
            plan = ram.plan_chunks(before, need, cached_row, W, layer * R, L * R)
            out[p + "ids"] = np.array(ids, np.int64)
            out[p + "need"] = need.numpy().copy()
            out[p + "before"] = before.numpy().copy()
            out[p + "cached_row"] = cached_row.numpy().copy()
            for name, arr in zip(("dst_row", "src_row", "maps", "todo", "ssd", "late"), plan):
                out[p + name] = arr.numpy().copy()
        state(p + "vram_", vram)
        state(p + "ram_", ram)
    return out


def main() -> None:
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    codec, table = _load_reference(root)
    np.savez_compressed(os.path.join(HERE, "codec_vectors.npz"), **codec_vectors(codec))
    small = table_vectors(table, E=16, S=3, R=6, W=3, L=2, layer=1, steps=120, seed=11)
    big = table_vectors(table, E=256, S=32, R=128, W=64, L=40, layer=7, steps=40, seed=12)
    np.savez_compressed(os.path.join(HERE, "table_vectors_small.npz"), **small)
    np.savez_compressed(os.path.join(HERE, "table_vectors_big.npz"), **big)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
