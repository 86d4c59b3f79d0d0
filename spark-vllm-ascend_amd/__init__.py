"""MI355X-native batch-1 Q4_0 decode path behind the Spark vLLM plugin hooks.

Layout (mirrors src/spark_vllm_ascend/ of the reference):
  plugin/       register(): vLLM general-plugin entry point (stdlib-only import)
  integration/  host side of the decode path: Q4_0 weight format, the Q4_0
                linear quant method, the split-KV attention backend, the
                per-layer decode step and the captured decode graph
  native/       the gfx950 HIP kernels and their C ABI (libsmx.so), bound
                with ctypes
"""

__version__ = "0.1.0"
