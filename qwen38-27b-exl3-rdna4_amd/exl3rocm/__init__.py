"""exl3rocm -- MI355X-native EXL3 quantized-linear engine (drop-in for the reference plugin's
linear path).  Submodules:

  ops      torch custom ops exl3rocm::linear / exl3rocm::linear_groups
  plugin   Exl3Config / Exl3LinearMethod (vLLM quantization surface)
  kernels  tensor wrappers of the C ABI (reference extension call names)
  layout   safetensors checkpoint layout discovery
  synth    seeded synthetic layers (counter RNG)
"""
__all__ = ["ops", "plugin", "kernels", "layout", "synth"]
