"""The drop-in boundary driven from C++ the way the AOT runtime would drive
it (tests/c_consumer/q8_consumer.cpp): an arena file is written, mapped and
registered with llmcp_q8_upload_arena, the default context is set, and the
_mlir_ciface_ entries are called with MemRef descriptors whose weight data
points into the mapping.  The data is llmcp-matmul-benchmark's Q8 fixture
(llmcp-matmul-benchmark.cpp:280-289, check :331-335: first == K), at its
registered 64x64x64 shape (tests/CMakeLists.txt:162-165) and on a decode-sized
256x2560 tensor, for M = 1 (decode GEMV) and M = 64 (prefill GEMM); then one
device-resident decode step (token id in HBM -> embedding -> lm_head -> argmax
id in HBM), where every logit ties and the first maximum must be row 0."""
import os
import subprocess
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from test_host import consumer_binary  # noqa: E402

pytestmark = pytest.mark.gpu


def test_cpp_consumer_arena_to_mlir_ciface(q8, tmp_path):
    q8.lib()  # fails loudly if the HIP library is missing
    print("q8_consumer --gpu", flush=True)
    r = subprocess.run([consumer_binary(), "--gpu", str(tmp_path)],
                       capture_output=True, text=True, timeout=100)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "device part ok" in r.stdout
    assert r.stdout.count("first") == 4
    assert "argmax 0" in r.stdout
