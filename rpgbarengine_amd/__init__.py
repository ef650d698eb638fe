"""MI355X-native Qwen3 token loop (HIP, gfx950) behind the RPGBarEngine C ABI."""
