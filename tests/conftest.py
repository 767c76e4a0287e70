import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vector-rs_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP library")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.lib()
    return o


@pytest.fixture(params=["direct", "mfma"])
def assign_path(request, monkeypatch):
    """k-means assignment path of the states a test creates: below 128 points per CU, with at most
    256 centroids, 1e6 (point, centroid) pairs and 1024 dimensions, squared L2, dot product and
    cosine take the direct form;
    VHIP_KMEANS_ASSIGN=mfma keeps them on the MFMA scan with its certified selection."""
    if request.param == "mfma":
        monkeypatch.setenv("VHIP_KMEANS_ASSIGN", "mfma")
    else:
        monkeypatch.delenv("VHIP_KMEANS_ASSIGN", raising=False)
    return request.param
