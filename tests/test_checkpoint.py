"""CPU: checkpoints in the reference's format (atlas_jax/train.py:86-131).

The reference writes Equinox's tree_serialise_leaves file: the model's array
leaves as consecutive .npy records, in the order JAX flattens the module
(dataclass fields in declaration order, static fields and None skipped).
These tests pin (1) the record format (standard .npy, read back one record
at a time with NumPy alone, bfloat16 as 2-byte void records), (2) a save /
load round trip into a differently initialised model, for the Atlas LM
(stacked blocks, persistent tokens) and the MAG transformer, (3) the
rejection of a checkpoint of another shape, and (4) when the reference
sources are present, the leaf order against the field declarations of the
reference's Equinox classes, read with `ast` (never imported)."""

import ast
import os

import numpy as np
import pytest
import torch

from atlas_amd import AtlasConfig
from atlas_amd import checkpoint as CK
from atlas_amd.mag import MAGTransformer
from atlas_amd.model import Atlas

REF = "/root/reference/atlas_jax"


def _cfg(**kw):
    c = dict(n_layer=2, n_embd=32, n_head=2, vocab_size=40, chunk_size=16, conv_kernel=2, ns_steps=3,
             omega_window=4, poly_degree=2, memory_expand=2, num_persist_mem_tokens=3, window_size=8)
    c.update(kw)
    return AtlasConfig(**c)


def _atlas(seed, **kw):
    return Atlas(_cfg(**kw), generator=torch.Generator().manual_seed(seed), device="cpu")


def _params(model):
    return {n: p.detach().clone() for n, p in model.named_parameters()}


def test_leaf_file_is_consecutive_npy_records(tmp_path):
    arrays = [torch.arange(6, dtype=torch.float32).reshape(2, 3), torch.tensor([1.5, -2.0]).bfloat16(),
              torch.zeros(0), np.int32(7)]
    path = tmp_path / "leaves.eqx"
    CK.write_leaves(path, arrays)
    with open(path, "rb") as f:
        recs = [np.load(f, allow_pickle=False) for _ in range(4)]
        assert f.read() == b""
    np.testing.assert_array_equal(recs[0], np.arange(6, dtype=np.float32).reshape(2, 3))
    assert recs[1].dtype.kind == "V" and recs[1].dtype.itemsize == 2
    # bfloat16 bits of 1.5 and -2.0
    np.testing.assert_array_equal(recs[1].view(np.uint16), np.array([0x3FC0, 0xC000], dtype=np.uint16))
    assert recs[2].shape == (0,) and recs[3] == 7
    back = CK.read_leaves(path)
    assert back[1].dtype == torch.bfloat16 and back[1].tolist() == [1.5, -2.0]
    assert torch.equal(back[0], arrays[0]) and int(back[3]) == 7


def test_atlas_round_trip(tmp_path):
    src, dst = _atlas(1), _atlas(2)
    before = _params(dst)
    CK.save_checkpoint(src, 123, tmp_path)
    assert sorted(os.listdir(tmp_path)) == ["meta.txt", "model.eqx"]
    step, opt = CK.load_checkpoint(dst, tmp_path)
    assert step == 123 and opt is None
    want = _params(src)
    for n, p in dst.named_parameters():
        assert torch.equal(p, want[n]), n
    # the two seeds differ in every randomly initialised tensor
    assert sum(not torch.equal(before[n], want[n]) for n in want) >= 20
    # the stacked layout: one record per block leaf with a leading n_layer axis
    leaves = CK.read_leaves(tmp_path / "model.eqx")
    names = [n for n, _ in CK.model_leaves(src)]
    assert names[0] == "wte.weight" and names[-2:] == ["lm_head.weight", "persist_mem"]
    i = names.index("blocks.memory.W1_init")
    assert leaves[i].shape == (2, 2, 16, 32)
    assert torch.equal(leaves[i][1], src.blocks[1].memory.W1_init.detach())


def test_round_trip_casts_dtype_and_keeps_optimizer_leaves(tmp_path):
    src = Atlas(_cfg(), generator=torch.Generator().manual_seed(3), device="cpu", dtype=torch.bfloat16)
    opt = [torch.ones(3), torch.tensor(5, dtype=torch.int32)]
    CK.save_checkpoint(src, 7, tmp_path, opt_leaves=opt)
    dst = _atlas(4)
    step, opt_back = CK.load_checkpoint(dst, tmp_path)
    assert step == 7 and torch.equal(opt_back[0], opt[0]) and int(opt_back[1]) == 5
    torch.testing.assert_close(dst.wte.weight, src.wte.weight.float(), rtol=0, atol=0)
    torch.testing.assert_close(dst.blocks[0].memory.c_q.weight, src.blocks[0].memory.c_q.weight.float(),
                               rtol=0, atol=0)


def test_mag_round_trip(tmp_path):
    cfg = _cfg(num_persist_mem_tokens=0, neural_memory_layers=(1,))
    src = MAGTransformer(cfg, generator=torch.Generator().manual_seed(5), device="cpu")
    dst = MAGTransformer(cfg, generator=torch.Generator().manual_seed(6), device="cpu")
    CK.save_checkpoint(src, 1, tmp_path)
    CK.load_checkpoint(dst, tmp_path)
    want = _params(src)
    for n, p in dst.named_parameters():
        assert torch.equal(p, want[n]), n
    names = [n for n, _ in CK.model_leaves(src)]
    assert "blocks.0.memory.W1_init" not in names and "blocks.1.memory.W1_init" in names
    assert names[1:4] == ["blocks.0.attn.to_qkv.weight", "blocks.0.attn.to_out.weight", "blocks.0.attn.rope.inv_freq"]


def test_load_rejects_other_shapes(tmp_path):
    CK.save_checkpoint(_atlas(1), 1, tmp_path)
    with pytest.raises(ValueError, match="leaves"):
        CK.load_checkpoint(_atlas(1, num_persist_mem_tokens=0), tmp_path)
    with pytest.raises(ValueError, match="shape"):
        CK.load_checkpoint(_atlas(1, n_embd=48), tmp_path)
    assert CK.load_checkpoint(_atlas(1), tmp_path / "absent") == (0, None)


# ---------------------------------------------------------------------------
# Leaf order against the reference's class declarations
# ---------------------------------------------------------------------------

def _dynamic_fields(path, cls):
    """Annotated fields of `cls` in declaration order, without the
    eqx.field(static=True) ones."""
    tree = ast.parse(open(path).read())
    for node in tree.body:
        if isinstance(node, ast.ClassDef) and node.name == cls:
            out = []
            for st in node.body:
                if isinstance(st, ast.AnnAssign) and isinstance(st.target, ast.Name):
                    static = (isinstance(st.value, ast.Call)
                              and any(k.arg == "static" and getattr(k.value, "value", False) for k in st.value.keywords))
                    if not static:
                        out.append(st.target.id)
            return out
    raise AssertionError(f"{cls} not in {path}")


def _collapse(names, depth):
    """Distinct consecutive name prefixes of `depth` dotted components."""
    out = []
    for n in names:
        key = ".".join(n.split(".")[:depth])
        if not out or out[-1] != key:
            out.append(key)
    return out


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference sources not present")
def test_leaf_order_follows_reference_field_order():
    ml = os.path.join(REF, "memory_layer.py")
    mo = os.path.join(REF, "model.py")
    mg = os.path.join(REF, "mag_transformer.py")
    mem_fields = _dynamic_fields(ml, "AtlasMemoryLayer")
    assert _dynamic_fields(ml, "ShortConv") == ["weight", "bias"]
    model = _atlas(1)
    mem = [n for n, _ in CK.memory_layer_leaves(model.blocks[0].memory)]
    assert _collapse(mem, 1) == mem_fields
    for n in mem:   # Linear and ShortConv leaves: weight before bias
        assert n.split(".")[-1] in ("weight", "bias") or "." not in n
    assert _dynamic_fields(mo, "Block") == ["memory", "mlp"]
    assert _dynamic_fields(mo, "MLP") == ["c_fc", "c_proj"]
    atlas_fields = _dynamic_fields(mo, "Atlas")
    assert atlas_fields == ["wte", "blocks", "lm_head", "persist_mem"]
    names = [n for n, _ in CK.model_leaves(model)]
    assert _collapse(names, 1) == atlas_fields
    assert _collapse([n for n in names if n.startswith("blocks.")], 2) == ["blocks.memory", "blocks.mlp"]

    assert _dynamic_fields(mg, "MAGTransformer") == ["wte", "blocks", "lm_head"]
    assert _dynamic_fields(mg, "MAGBlock") == ["attn", "memory", "gate", "mlp"]
    assert _dynamic_fields(mg, "MemoryGate") == ["linear"]
    assert _dynamic_fields(mo, "SlidingWindowAttention") == ["norm", "to_qkv", "to_out", "rope"]
    assert _dynamic_fields(mo, "RotaryEmbedding") == ["inv_freq"]
    mag = MAGTransformer(_cfg(num_persist_mem_tokens=0), generator=torch.Generator().manual_seed(5), device="cpu")
    names = [n for n, _ in CK.model_leaves(mag)]
    blk0 = [n[len("blocks.0."):] for n in names if n.startswith("blocks.0.")]
    # norm is None in the reference (no leaf)
    assert _collapse(blk0, 1) == ["attn", "memory", "gate", "mlp"]
    assert _collapse([n for n in blk0 if n.startswith("attn.")], 2) == ["attn.to_qkv", "attn.to_out", "attn.rope"]


def test_model_only_save_removes_stale_optimizer_file(tmp_path):
    """A save without optimiser leaves over a directory that holds an older
    opt_state.eqx removes it (a load must not pair it with the newer model)
    and warns that the directory is not loadable by the reference, whose
    load_checkpoint always reads opt_state.eqx (train.py:121-122)."""
    import pytest
    src = _atlas(1)
    CK.save_checkpoint(src, 5, tmp_path, opt_leaves=[torch.ones(2)])
    assert sorted(os.listdir(tmp_path)) == ["meta.txt", "model.eqx", "opt_state.eqx"]
    with pytest.warns(UserWarning, match="opt_state.eqx"):
        CK.save_checkpoint(src, 9, tmp_path)
    assert sorted(os.listdir(tmp_path)) == ["meta.txt", "model.eqx"]
    step, opt = CK.load_checkpoint(_atlas(2), tmp_path)
    assert step == 9 and opt is None
