"""The reference's 19 integration tests, ported onto the C++ front end
(katsu_amd/cpp) and run by the driver tests/cpp/_build/test_frontend.

The front end keeps tensor data, adjoints and gradients on the GPU, so every
test that computes needs it; the shape-validation tests run anywhere.  The
driver is run once per session; each test checks its line."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "tests", "cpp", "_build", "test_frontend")

# No kernel launch (shape and length validation only): runnable without a GPU.
HOST_ONLY = [
    "validates_data_and_storage_size",
    "scalar_and_empty_shapes",
    "rejects_invalid_matmul",
]
# Compute on the GPU: every op, adjoint and gradient of the front end is
# device-resident.
DEVICE = [
    "addition_preserves_inputs",
    "empty_matmul_and_output_overflow",
    "squared_error_shared_nodes_and_repeated_backward",
    "diamond_and_clone_identity",
    "explicit_seed_and_errors_are_atomic",
    "empty_graph_operations",
    "empty_batch_and_seeded_initialization",
    "rectangular_matmul",
    "matmul_finite_differences",
    "matmul_same_parent_accumulates_both_edges",
    "known_forward_and_overlap_gradients",
    "finite_differences_input_and_weights",
    "reused_layer_keeps_independent_graphs",
    "shared_operand_and_chained_convolution",
    "invalid_shapes_and_overflow",
    "known_stride_and_padding",
]
# The device engine's own features (no counterpart test in the reference).
EXTRA_DEVICE = [
    "stem_chain_on_device",
    "grad_cam_on_device",
    "grad_cam_resized_to_input",
    "publish_is_all_or_nothing",
]


def _driver():
    if not os.path.exists(DRIVER):
        sys.path.insert(0, os.path.join(ROOT, "tests", "cpp"))
        import build as cpp_build  # noqa: E402
        cpp_build.build()
    return DRIVER


def _run(names):
    proc = subprocess.run([_driver(), *names], capture_output=True, text=True, timeout=600)
    results = {}
    for line in proc.stdout.splitlines():
        status, _, rest = line.partition(" ")
        name = rest.split(":", 1)[0]
        results[name] = (status, line)
    return results


@pytest.fixture(scope="module")
def host_results():
    return _run(HOST_ONLY)


@pytest.fixture(scope="module")
def device_results():
    return _run(DEVICE + EXTRA_DEVICE)


def test_every_reference_test_is_ported():
    assert len(HOST_ONLY) + len(DEVICE) == 19
    assert not set(HOST_ONLY) & set(DEVICE)


@pytest.mark.parametrize("name", HOST_ONLY)
def test_frontend_host(name, host_results):
    status, line = host_results.get(name, ("MISSING", name))
    assert status == "PASS", line


@pytest.mark.gpu
@pytest.mark.parametrize("name", DEVICE + EXTRA_DEVICE)
def test_frontend_device(name, device_results):
    status, line = device_results.get(name, ("MISSING", name))
    assert status == "PASS", line


def test_seeded_weights_match_repo_example():
    """Conv2D::new_seeded(3, 8, (3, 3), 1, 1, 123), the repository example's
    layer (examples/conv2d/main.rs:9), bit for bit against the weights the
    oracle's restatement of conv2d.rs:35-61 wrote into
    tests/golden/example_1b.json (host-side: no device call)."""
    import json

    import numpy as np
    ref = json.load(open(os.path.join(ROOT, "tests", "golden", "example_1b.json")))["w"]
    want = np.array(ref, np.float32).view(np.uint32)
    proc = subprocess.run([_driver(), "--seeded-weights", "3", "8", "3", "3", "123"],
                          capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    got = np.array([int(v, 16) for v in proc.stdout.split()], np.uint32)
    assert got.shape == want.shape == (216,)
    assert np.array_equal(got, want)
    # And the oracle's own generator, on a second seed and shape.
    proc = subprocess.run([_driver(), "--seeded-weights", "5", "4", "2", "3", "7"],
                          capture_output=True, text=True, timeout=60)
    got = np.array([int(v, 16) for v in proc.stdout.split()], np.uint32)
    from oracle import oracle as O
    assert np.array_equal(got, O.seeded_weights(5, 4, (2, 3), 7).ravel().view(np.uint32))
