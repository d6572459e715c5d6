"""One GPU's share of the LLaMA decode step under 8-way tensor parallelism:
the decode-step spec (llama_decoder_step.py, reference
mlx/kernels/full/llama_decoder_layer.py:24-64) on the shard's matrices --
4 of the 32 query heads and 1 of the 8 KV heads, the matching 512 rows of
W_o, 1792 of the 14336 gate / up columns and W_down rows.  It measures one
shard's work at its real shapes and is not a tensor-parallel decomposition:
the step adds the full residual x and normalises its own partial
x1 = x + attn @ W_o, so the shards' y do not sum to the layer's output (a
real shard splits the step at W_o, all-reduces attn @ W_o between the
halves and adds each residual on one rank).  Run on the host CPU in fp32."""
import importlib.util
from pathlib import Path

# The same Model as the whole-layer entry; the registry's model_kwargs give
# the shard's shapes.
_path = Path(__file__).with_name("llama_decoder_step.py")
_spec = importlib.util.spec_from_file_location("_mb_llama_decoder_step_for_tp8", _path)
_mod = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(_mod)
Model = _mod.Model
