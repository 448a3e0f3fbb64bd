"""TEST-ONLY stand-in for the parts of vLLM the plugin touches (vLLM is not installed in
this image).  It mirrors the upstream interfaces the reference plugin relies on:
PluggableLayer.register_oot, LogitsProcessor._get_logits, VocabParallelEmbedding,
vllm.v1.sample.sampler.Sampler(.sample), SamplingMetadata and LogitsProcessors."""
