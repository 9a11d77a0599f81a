"""The round-end smoke check (`__graft_entry__.smoke()`) runs green: one tiled
transpose and one split sum on the GPU, bit-identical to the CPU oracle."""
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))


def test_smoke_matches_the_oracle():
    import __graft_entry__ as entry
    entry.smoke()
