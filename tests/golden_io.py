"""(De)serialisation of small decode cases for tests/golden/ (npz, no pickle)."""
import numpy as np

from oracle.attention import ColdBlock, TierState


def save_decode_case(path, Q, state, cos, sin, q, **extra):
    arrs = {"Q": Q, "cos": cos, "sin": sin, "q": np.array(q), "nblk": np.array(len(state.blocks))}
    for j, b in enumerate(state.blocks):
        for name in ("codes_k", "scale_k", "basis_k", "codes_v", "scale_v", "basis_v"):
            arrs[f"b{j}_{name}"] = getattr(b, name)
        arrs[f"b{j}_start"] = np.array(b.start)
    if state.tail_len:
        arrs["tail_k"], arrs["tail_v"], arrs["tail_pos"] = state.tail_k, state.tail_v, np.asarray(state.tail_pos)
    arrs.update(extra)
    np.savez_compressed(path, **arrs)


def load_decode_case(path):
    g = np.load(path, allow_pickle=False)
    blocks = []
    for j in range(int(g["nblk"])):
        blocks.append(ColdBlock(g[f"b{j}_codes_k"], g[f"b{j}_scale_k"], g[f"b{j}_basis_k"], g[f"b{j}_codes_v"],
                                g[f"b{j}_scale_v"], g[f"b{j}_basis_v"], int(g[f"b{j}_start"])))
    tail = (g["tail_k"], g["tail_v"], g["tail_pos"]) if "tail_k" in g else (None, None, None)
    out = {k: g[k] for k in g.files}
    out["state"] = TierState(blocks, *tail)
    out["q"] = int(g["q"])
    return out
