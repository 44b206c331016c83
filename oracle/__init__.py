"""CPU oracle of the expert-paging hot path -- TEST INFRASTRUCTURE ONLY.

Plain restatements of the reference algorithm (monochromegane/vllm-expert-pager
v0.1.1), used as the checker by tests/, by __graft_entry__.smoke() and by the
cpu_baseline leg of bench.py. The product (vllm-expert-pager_amd/) never
imports, links or runs anything here.

Modules:
  table_ref  -- LRU tables: need_mask, acquire, pack, seed, plan_chunks
                (table.py:28-247), plus an independent dict-based LRU
                (tests/test_table.py:13-51) used to pin acquire.
  codec_ref  -- row codec: code_lengths / Code / encode (codec.py:61-198) and
                the sequential decoder rule (tests/test_codec.py:49-79); a C
                build of the decoder (codec_ref.c) for large rows and the CPU
                baseline.
  gather_ref -- byte semantics of gather_rows / decode_rows (gather.py:328-393,
                codec.py:297-327) and the chunk-loop simulator
                (tests/test_table.py:200-281).
  moe_ref    -- fp32 restatement of the block-fp8 expert FFN and the single
                top-k combine used on the prefill overflow path.

Pinning status of each function is stated in its module docstring.
"""
