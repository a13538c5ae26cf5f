"""Hugging Face model integrations (reference models/): Llama and Qwen2."""
