import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm GPU) and the built libattnnn.so")


@pytest.fixture(scope="session")
def tiny_cfg():
    from attention_nn_amd.config import GPTConfig
    # the reference's own tiny self-test config (model.py:290-291)
    return GPTConfig(vocab_size=512, num_layers=2, num_heads=4, model_dim=64, seq_len=32,
                     window=16, long_layers=(1,))
