"""MI355X-native attention + speculative-verify hot path for nano-vllm-spec-decode.

Drop-in modules mirroring the reference layout:
  nanovllm_amd.layers.attention  <-> nanovllm/layers/attention.py  (store_kvcache, Attention)
  nanovllm_amd.layers.sampler    <-> nanovllm/layers/sampler.py    (verify_drafts, Sampler)
  nanovllm_amd.utils.context     <-> nanovllm/utils/context.py     (Context, set/get/reset_context)
  nanovllm_amd.engine.metadata   <-> batch layout builders of nanovllm/engine/model_runner.py
The compute runs in libsd_attn.so (HIP, gfx950); see _lib.py.
"""
