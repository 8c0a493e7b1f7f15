"""MI355X-native implementation of AxiomLM's quantized decode step.

Sub-modules:
  kernels      -- ``axiomlm.kernels``-compatible operators (HIP, libaxm.so)
  cache        -- ``StaticKVCache`` (fp16 / FP8 / INT4, ring buffer)
  runner       -- ``QuantizedDecodeRunner`` (whole-step hipGraph)
  transformer  -- ``ModelConfig`` / ``Transformer`` decode driver
  build        -- ahead-of-time hipcc build of libaxm.so
"""

__version__ = "0.1.0"
