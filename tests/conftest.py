import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def tune():
    """Planner overrides through fkv_set_tuning for one test: tune(attn_order=0,
    attn_stream=1, attn_split_tokens=..., prefill_split_blocks=..., attn_engine=1,
    attn_wgs_per_cu=2); every knob the test
    set goes back to the planner's own rule afterwards."""
    import ferrum_amd as fa
    knobs = {"attn_split_tokens": (fa.TUNE_ATTN_SPLIT_TOKENS, 0),
             "attn_stream": (fa.TUNE_ATTN_STREAM, 0),
             "attn_order": (fa.TUNE_ATTN_ORDER, -1),
             "prefill_split_blocks": (fa.TUNE_PREFILL_SPLIT_BLOCKS, -1),
             "attn_engine": (fa.TUNE_ATTN_ENGINE, 0),
             "attn_wgs_per_cu": (fa.TUNE_ATTN_WGS_PER_CU, 0)}
    touched = set()

    def set_knobs(**kw):
        for name, value in kw.items():
            fa.set_tuning(knobs[name][0], int(value))
            touched.add(name)
    yield set_knobs
    for name in touched:
        fa.set_tuning(*knobs[name])
