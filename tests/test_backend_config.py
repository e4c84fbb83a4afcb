"""AttentionConfig as the reference's own tests check it
(attention/backend.rs:317-344), through the C ABI (no GPU needed)."""
import math

import numpy as np

from dendrite_amd.backend import AttentionConfig


def test_attention_config_defaults():
    config = AttentionConfig.default()
    assert (config.num_heads, config.num_kv_heads, config.head_dim) == (8, 8, 64)
    assert config.sliding_window is None


def test_attention_config_scale():
    config = AttentionConfig.new(8, 8, 64)
    assert abs(config.scale - 1.0 / math.sqrt(64.0)) < 1e-6
    assert config.scale == float(np.float32(1.0) / np.sqrt(np.float32(64.0)))


def test_attention_config_sliding_window():
    config = AttentionConfig.new(8, 8, 64).with_sliding_window(4096)
    assert config.sliding_window == 4096


def test_attention_config_gqa():
    config = AttentionConfig.new(32, 8, 128)
    assert config.num_queries_per_kv() == 4
