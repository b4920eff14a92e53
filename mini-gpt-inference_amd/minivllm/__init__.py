"""minivllm for MI355X: the paged-KV decode hot path of the Mini-GPT runtime.

Same module layout and API as the reference ``minivllm`` package
(``KVBlockPool``, ``BlockManager``, ``DecodeBatchMetadata``,
``ModelRunner.decode_batch``, ``MiniGPT.set_decode_attention_backend``), with
the decode KV append and paged decode attention running as hand-written HIP
kernels for gfx950 (``minivllm.hip_paged_decode``) behind the C ABI of
``libminivllm_hip.so``.
"""
