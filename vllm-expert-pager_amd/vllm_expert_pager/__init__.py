"""MI355X-native expert paging for vLLM (drop-in for monochromegane/vllm-expert-pager).

Host side of the GPU paging hot path: LRU slot tables, slot gather from the
pinned RAM tier, per-row fp8 exponent Huffman expansion and the prefill
overflow path. The kernels live in libxp.so (gfx950 HIP, built from csrc/).
"""

__version__ = "0.1.0"
