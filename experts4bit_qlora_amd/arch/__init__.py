"""Architecture-specific expert epilogues (DeepSeek-V4 clamped SwiGLU, gpt-oss clamped GLU)."""
