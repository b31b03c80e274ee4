"""Text facades over the engine (LLM, AsyncLLM)."""
