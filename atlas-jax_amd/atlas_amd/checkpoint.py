"""Model checkpoints in the reference's on-disk format (atlas_jax/train.py:86-131).

The reference saves `model.eqx` and `opt_state.eqx` with Equinox's
`tree_serialise_leaves` and the step in `meta.txt`, renaming temporary files
into place so that a crash never leaves a half-written checkpoint.  The leaf
file is the model's array leaves, one NumPy `.npy` record after another, in
the order JAX flattens the Equinox module: dataclass fields in declaration
order, static fields skipped, `None` fields contributing nothing, lists in
order.  bfloat16 leaves are stored as 2-byte void records (NumPy has no
bfloat16 type).

This module writes and reads that format for `Atlas` and `MAGTransformer`:
the leaf order below is the reference's field order, mapped to this
package's parameter names.
  - Atlas (model.py:271-277): wte.weight, then every leaf of the stacked
    blocks (Block, model.py:174-177: memory, mlp) with a leading n_layer
    axis, lm_head.weight, persist_mem.
  - AtlasMemoryLayer (memory_layer.py:347-375): c_q, c_k, c_v, c_proj
    (weights only), conv_q/k/v (weight, bias), gate_alpha/eta/theta (weight,
    bias), gate_gamma (when Omega > 1), poly_coeffs (degree > 0), ln_gamma,
    W1_init, W2_init, retrieve_gate (H > 1).
  - MLP (model.py:142-146): c_fc.weight, c_proj.weight.
  - MAGTransformer (mag_transformer.py:88-92): wte.weight, the blocks in
    order (not stacked), lm_head.weight; MAGBlock (:37-40): attn
    (SlidingWindowAttention, model.py:79-82: to_qkv.weight, to_out.weight,
    rope.inv_freq), memory, gate (MemoryGate.linear weight and bias), mlp.
Only the model file is mapped to parameters; the optimiser file's leaves are
returned as a list (its tree is optax's state, which has no counterpart
here), and `save_checkpoint` writes one only when given such a list.
"""

import os
import warnings

import numpy as np
import torch

_BF16_VOID = np.dtype("V2")


# ---------------------------------------------------------------------------
# The leaf file
# ---------------------------------------------------------------------------

def _to_numpy(t):
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(_BF16_VOID)
    return t.numpy()


def _to_torch(a):
    if a.dtype.kind == "V" and a.dtype.itemsize == 2:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(np.array(a, copy=True))


def write_leaves(path, arrays):
    """One .npy record per array, in order (tree_serialise_leaves' file)."""
    with open(path, "wb") as f:
        for a in arrays:
            np.save(f, _to_numpy(a) if isinstance(a, torch.Tensor) else np.asarray(a), allow_pickle=False)


def read_leaves(path):
    """Every .npy record of a leaf file, in order, as torch tensors (CPU).
    Nothing in the file is unpickled."""
    out = []
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        while f.tell() < size:
            out.append(_to_torch(np.load(f, allow_pickle=False)))
    return out


# ---------------------------------------------------------------------------
# Leaf order of the reference modules, as this package's parameters
# ---------------------------------------------------------------------------

def memory_layer_leaves(mem):
    """(name, tensor) of one AtlasMemoryLayer in the reference's field order."""
    out = [("c_q.weight", mem.c_q.weight), ("c_k.weight", mem.c_k.weight), ("c_v.weight", mem.c_v.weight),
           ("c_proj.weight", mem.c_proj.weight)]
    for c in "qkv":
        conv = getattr(mem, "conv_" + c)
        out += [(f"conv_{c}.weight", conv.weight), (f"conv_{c}.bias", conv.bias)]
    for g in ("alpha", "eta", "theta", "gamma"):
        lin = getattr(mem, "gate_" + g)
        if lin is not None:
            out += [(f"gate_{g}.weight", lin.weight), (f"gate_{g}.bias", lin.bias)]
    if mem.poly_coeffs is not None:
        out.append(("poly_coeffs", mem.poly_coeffs))
    out += [("ln_gamma", mem.ln_gamma), ("W1_init", mem.W1_init), ("W2_init", mem.W2_init)]
    if mem.retrieve_gate is not None:
        out.append(("retrieve_gate.weight", mem.retrieve_gate.weight))
    return out


def _mlp_leaves(mlp):
    return [("c_fc.weight", mlp.c_fc.weight), ("c_proj.weight", mlp.c_proj.weight)]


def model_leaves(model):
    """The checkpoint's leaves of `model` as (name, [tensors]) in file order:
    one tensor per leaf, or for Atlas's stacked blocks one tensor per layer
    (stacked along a new leading axis in the file)."""
    from .mag import MAGTransformer
    from .model import Atlas
    if isinstance(model, Atlas):
        out = [("wte.weight", [model.wte.weight])]
        per_layer = []
        for blk in model.blocks:
            per_layer.append([("memory." + n, t) for n, t in memory_layer_leaves(blk.memory)]
                             + [("mlp." + n, t) for n, t in _mlp_leaves(blk.mlp)])
        for i, (name, _) in enumerate(per_layer[0]):
            out.append(("blocks." + name, [layer[i][1] for layer in per_layer]))
        out.append(("lm_head.weight", [model.lm_head.weight]))
        if model.persist_mem is not None:
            out.append(("persist_mem", [model.persist_mem]))
        return out
    if isinstance(model, MAGTransformer):
        out = [("wte.weight", [model.wte.weight])]
        for li, blk in enumerate(model.blocks):
            pre = f"blocks.{li}."
            out += [(pre + "attn.to_qkv.weight", [blk.attn.to_qkv.weight]),
                    (pre + "attn.to_out.weight", [blk.attn.to_out.weight]),
                    (pre + "attn.rope.inv_freq", [blk.attn.rope.inv_freq])]
            if blk.memory is not None:
                out += [(pre + "memory." + n, [t]) for n, t in memory_layer_leaves(blk.memory)]
                out += [(pre + "gate.linear.weight", [blk.gate.linear.weight]),
                        (pre + "gate.linear.bias", [blk.gate.linear.bias])]
            out += [(pre + "mlp." + n, [t]) for n, t in _mlp_leaves(blk.mlp)]
        out.append(("lm_head.weight", [model.lm_head.weight]))
        return out
    raise TypeError(f"no checkpoint layout for {type(model).__name__}")


def _stacked(ts):
    return ts[0].detach() if len(ts) == 1 else torch.stack([t.detach() for t in ts])


def state_arrays(model):
    """The model's leaves as the checkpoint stores them (CPU tensors)."""
    return [_stacked(ts).cpu() for _, ts in model_leaves(model)]


def load_arrays(model, arrays):
    """Copy checkpoint leaves (file order) into `model`'s parameters, casting
    to each parameter's dtype.  Raises ValueError on a count or shape
    mismatch (the reference's tree_deserialise_leaves raises on those too)."""
    leaves = model_leaves(model)
    if len(arrays) != len(leaves):
        raise ValueError(f"checkpoint holds {len(arrays)} leaves, the model has {len(leaves)}")
    with torch.no_grad():
        for (name, ts), a in zip(leaves, arrays):
            want = tuple(ts[0].shape) if len(ts) == 1 else (len(ts), *ts[0].shape)
            if tuple(a.shape) != want:
                raise ValueError(f"leaf {name}: checkpoint shape {tuple(a.shape)}, model {want}")
            if len(ts) == 1:
                ts[0].copy_(a.to(ts[0].dtype))
            else:
                for i, t in enumerate(ts):
                    t.copy_(a[i].to(t.dtype))


# ---------------------------------------------------------------------------
# Checkpoint directory (train.py:86-131)
# ---------------------------------------------------------------------------

def save_checkpoint(model, step, ckpt_dir, opt_leaves=None):
    """Write model.eqx (and opt_state.eqx when opt_leaves is given) and
    meta.txt into ckpt_dir through temporary files renamed into place.

    Without opt_leaves any opt_state.eqx already in ckpt_dir (from an earlier
    save) is removed, so that a later load never pairs it with the newer
    model.  Such a directory holds no optimiser file, which the reference's
    load_checkpoint always reads (train.py:121-122): it resumes here, not
    there (a warning says so)."""
    os.makedirs(ckpt_dir, exist_ok=True)
    if opt_leaves is None:
        stale = os.path.join(ckpt_dir, "opt_state.eqx")
        if os.path.exists(stale):
            os.remove(stale)
        warnings.warn("save_checkpoint without opt_leaves writes no opt_state.eqx: the directory cannot be "
                      "loaded by the reference's load_checkpoint (train.py:121-122)", stacklevel=2)
    tmp_model = os.path.join(ckpt_dir, "model.eqx.tmp")
    tmp_opt = os.path.join(ckpt_dir, "opt_state.eqx.tmp")
    tmp_meta = os.path.join(ckpt_dir, "meta.tmp")
    write_leaves(tmp_model, state_arrays(model))
    if opt_leaves is not None:
        write_leaves(tmp_opt, opt_leaves)
    with open(tmp_meta, "w") as f:
        f.write(f"{int(step)}\n")
    os.replace(tmp_model, os.path.join(ckpt_dir, "model.eqx"))
    if opt_leaves is not None:
        os.replace(tmp_opt, os.path.join(ckpt_dir, "opt_state.eqx"))
    os.replace(tmp_meta, os.path.join(ckpt_dir, "meta.txt"))


def load_checkpoint(model, ckpt_dir):
    """Load model.eqx into `model` in place.  Returns (step, opt_leaves):
    step 0 and None when ckpt_dir holds no checkpoint (the reference returns
    its inputs unchanged then); opt_leaves is the optimiser file's leaves, or
    None when there is none."""
    model_path = os.path.join(ckpt_dir, "model.eqx")
    if not os.path.exists(model_path):
        return 0, None
    load_arrays(model, read_leaves(model_path))
    opt_path = os.path.join(ckpt_dir, "opt_state.eqx")
    opt = read_leaves(opt_path) if os.path.exists(opt_path) else None
    with open(os.path.join(ckpt_dir, "meta.txt")) as f:
        step = int(f.read().strip())
    return step, opt
