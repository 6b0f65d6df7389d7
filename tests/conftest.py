import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP library")


@pytest.fixture(scope="session")
def hip():
    """The HIP library bound through ctypes (fails loudly when it is not built)."""
    import infengine_amd
    return infengine_amd


@pytest.fixture(scope="session")
def ctx():
    import torch
    from infengine_amd.engine import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, graph=False)
    yield c
    torch.cuda.synchronize()
    c.close()


@pytest.fixture(autouse=True)
def _gpu_stream(request):
    """GPU tests run torch and the library on the session context's stream."""
    if request.node.get_closest_marker("gpu") is None:
        yield
        return
    import torch
    import gpu_util
    c = request.getfixturevalue("ctx")
    torch.cuda.synchronize()
    torch.cuda.set_stream(c.stream)
    yield
    torch.cuda.synchronize()
    gpu_util.release()
    # hand torch's cached blocks back to the device: the library allocates with hipMalloc
    # (weights arenas, page pools), which torch's cache would otherwise crowd out over a session
    torch.cuda.empty_cache()


# ---------------------------------------------------------------- the full random-init model
MODEL_SEED = 2024      # ie_model_weights_random_init(seed) and oracle.SyntheticModel(seed)
NOISE_POS = 300        # decode position the summation-order noise floor is measured at


@pytest.fixture(scope="session")
def model():
    """The full 32-layer random-init Llama-3.1-8B on the GPU (16 GB), shared by the modules."""
    import torch
    from gpu_util import say
    from infengine_amd.engine import ModelWeights
    say("random_init full model (16 GB) on the GPU")
    W = ModelWeights.random_init(seed=MODEL_SEED, std=0.02)
    torch.cuda.synchronize()
    yield W
    torch.cuda.synchronize()
    W.free()


@pytest.fixture(scope="session")
def oracle_model():
    import oracle as orc
    return orc.SyntheticModel(MODEL_SEED, 0.02)


@pytest.fixture(scope="session")
def noise_floor(oracle_model):
    """The 32-layer stack's own fp32 rounding-noise floor: the oracle's decode logits with every
    dot product summed in ascending vs descending order (max of max-abs/scale and mean-rel)."""
    import numpy as np
    import oracle as orc
    from gpu_util import say
    from tolerance import rel_errors
    say("oracle noise floor: ascending vs descending fp32 summation, 32 layers")
    prior = orc.synthetic((32, 2, 8, NOISE_POS, 128), MODEL_SEED, 900, 0.0, 1.0)
    kv = np.zeros((32, 2, 8, NOISE_POS + 2, 128), np.uint16)
    kv[:, :, :, :NOISE_POS] = prior
    a = oracle_model.decode(4242, NOISE_POS, kv)
    kv[:, :, :, NOISE_POS:] = 0
    with orc.reversed_summation():
        b = oracle_model.decode(4242, NOISE_POS, kv)
    mx, mean = rel_errors(b, a)
    say(f"noise floor: max-abs/scale {mx:.3e}, mean-rel {mean:.3e}")
    return max(mx, mean)
