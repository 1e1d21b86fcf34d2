import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "sparse-computation_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "sparse-computation_amd", "code_gen"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

REF_MATRICES = "/root/reference/matrices"
FIXTURE_STEM = "body_decoder_layer_1_encdec_attention_multihead_attention_k_fully_connected"
# The reference's fixture matrix (values 1, 512 x 512) and its km 4 x kn 2
# .cfmtx, committed gzipped: data files of the reference's own tree, so the
# GPU box (where the reference is not mounted) runs on the same matrix.
GOLDEN_MATRIX = os.path.join(ROOT, "tests", "golden", "reference_matrix")
GOLDEN_FILES = (FIXTURE_STEM + ".mtx", FIXTURE_STEM + "-4-2.cfmtx")


@pytest.fixture(scope="session")
def reference_matrix_dir(tmp_path_factory):
    """A directory holding the committed reference fixture files, unpacked."""
    import gzip
    import shutil
    d = tmp_path_factory.mktemp("reference_matrix")
    for name in GOLDEN_FILES:
        with gzip.open(os.path.join(GOLDEN_MATRIX, name + ".gz"), "rb") as src, open(d / name, "wb") as dst:
            shutil.copyfileobj(src, dst)
    return str(d)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no HIP device in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
