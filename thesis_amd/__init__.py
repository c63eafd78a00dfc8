"""MI355X-native packed ragged LayerSkip-Llama forward (the hot path of hsungo/thesis).

Host code is Python on PyTorch-ROCm (device memory, streams); every operation of the packed forward
and its step glue runs in liblsk.so, hand-written gfx950 HIP kernels behind a C ABI (include/lsk.h).

  thesis_amd.common.model       LayerSkipLlama, ModelConfig, KVCache (common/model.py surface)
  thesis_amd.common.engine      DecodeEngine, ARBatchEngine, SyncSpecEngine (common/engine.py surface)
  thesis_amd.common.methods     MethodSpec / register / METHODS (common/methods.py surface)
  thesis_amd.solutions.packed   Block, PackedBatch, build_packed, packed_layer(s) (solutions/packed.py)
  thesis_amd.solutions.engine   EESDEngine (solutions/engine.py surface)
"""

__version__ = "0.1.0"
