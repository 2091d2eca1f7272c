"""MI355X-native Delta Attention prefill path.

Public surface (mirrors the reference package `delta_attention`):
  delta_kernel.attention      query-sparse / key-dense attention
  stride.apply_delta_variable variable-stride delta broadcast
  llama.LlamaAttention        delta_forward / hip_attention_interface
  qwen3.Qwen3DeltaAttention   Qwen3 q/k-norm prologue
  config.Config, PIPELINE_FIELDS
  ops                         torch-level wrappers of the C ABI
"""

from ._lib import ExtensionMissing, LIB_PATH  # noqa: F401
