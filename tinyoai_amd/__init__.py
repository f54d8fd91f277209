"""tinyoai_amd: an MI355X (gfx950) HIP backend for tinyoai's StableLM/Llama forward pass."""
