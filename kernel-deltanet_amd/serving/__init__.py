"""Reference-named serving surfaces of the path on MI355X (reference serving/): the ragged mixed
prefill + decode step over resident states and the slab state pool, on the gfx950 kernels of libkdn.so."""
from .hybrid_memory_pool import HybridMemoryPool
from .vllm_kernel_deltanet_op import fork_recurrent_state, hybrid_recurrent_forward

__all__ = ["HybridMemoryPool", "hybrid_recurrent_forward", "fork_recurrent_state"]
