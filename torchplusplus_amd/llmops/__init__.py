"""LLM runtime mirroring torchpp.llmops (reference: torchpp/llmops/)."""
