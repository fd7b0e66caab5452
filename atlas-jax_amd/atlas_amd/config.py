"""AtlasConfig: the hyper-parameters the memory layer and model read.

Field names, meanings and defaults follow the reference's AtlasConfig
(atlas_jax/config.py:6-33) so configs carry over unchanged.  Two fields are
added: `scan_precision` selects the arithmetic of the HIP scan ("f32": fp32
MFMA throughout; "f16": fp16 MFMA operands with fp32 accumulation and fp32
state; None: "f32" for fp32 activations, "f16" otherwise) when no gradient
is taken, `scan_backward` the training path of the scan ("hip": the
library's atlas_scan_bwd; "torch": the inner gradient as differentiable
torch ops around the fused-chunk operator; None: "hip" where it is
compiled), and `scan_train_precision` the arithmetic of that library
training path ("f16": forward on fp16 matrix-core operands keeping its
chunk-start states, Polar-Express and its VJP on fp16 operands -- the only
library backward for E = 256; None / "f32": fp32).
"""

from dataclasses import dataclass


@dataclass
class AtlasConfig:
    sequence_len: int = 2048
    vocab_size: int = 32768
    n_layer: int = 24
    n_head: int = 16
    n_embd: int = 1536
    dim_head: int | None = None
    chunk_size: int = 64
    conv_kernel: int = 4
    ns_steps: int = 5
    omega_window: int = 16
    poly_degree: int = 2
    deep_memory: bool = True
    memory_expand: int = 2
    pe_ste: bool = False
    use_checkpoint: bool = True
    fused_chunk: bool = False
    dropout: float = 0.0
    gate_bias_init: float = 0.0
    max_lr: float = 0.1
    logit_softcap: float = 0.0
    num_persist_mem_tokens: int = 0
    stop_grad_chunks: bool = False
    geglu_ff: bool = True
    window_size: int = 64
    neural_memory_layers: tuple | None = None
    scan_precision: str | None = None
    scan_backward: str | None = None
    scan_train_precision: str | None = None

    @property
    def head_dim(self) -> int:
        return self.dim_head if self.dim_head is not None else self.n_embd // self.n_head

    @property
    def expand_dim(self) -> int:
        return self.memory_expand * self.head_dim if self.deep_memory else self.head_dim
