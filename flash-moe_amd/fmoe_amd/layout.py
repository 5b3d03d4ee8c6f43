"""Expert blob layout (config.h:94-137 compute_expert_offsets) in Python.

Nine tensors per expert, in the order gate_w, gate_s, gate_b, up_w, up_s,
up_b, down_w, down_s, down_b.  W rows hold ceil(in / (32/bits)) uint32 words;
scale/bias rows hold ceil(in / group_size) bf16 values.
"""
TENSORS = ("gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b")


def expert_offsets(hidden, inter, group_size, bits):
    """Returns (offsets dict, blob size in bytes)."""
    per = 32 // bits
    gw = inter * ((hidden + per - 1) // per) * 4
    gsz = inter * ((hidden + group_size - 1) // group_size) * 2
    dw = hidden * ((inter + per - 1) // per) * 4
    dsz = hidden * ((inter + group_size - 1) // group_size) * 2
    sizes = (gw, gsz, gsz, gw, gsz, gsz, dw, dsz, dsz)
    off, o = {}, 0
    for name, s in zip(TENSORS, sizes):
        off[name] = o
        o += s
    return off, o


def tensor_shapes(hidden, inter, group_size, bits):
    """(dtype-name, shape) of each tensor."""
    per = 32 // bits
    return {
        "gate_w": ("u32", (inter, hidden // per)), "gate_s": ("u16", (inter, hidden // group_size)),
        "gate_b": ("u16", (inter, hidden // group_size)),
        "up_w": ("u32", (inter, hidden // per)), "up_s": ("u16", (inter, hidden // group_size)),
        "up_b": ("u16", (inter, hidden // group_size)),
        "down_w": ("u32", (hidden, inter // per)), "down_s": ("u16", (hidden, inter // group_size)),
        "down_b": ("u16", (hidden, inter // group_size)),
    }
