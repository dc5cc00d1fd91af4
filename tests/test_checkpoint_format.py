"""numrs's JSON checkpoint format, on the CPU.

The document is serde_json of {model: OnnxModel, training_state: TrainingState}
(ops/model.rs:544-588, llo/model.rs): the reader is checked on a document laid
out field by field as those serde derives write it (the reference ships no
checkpoint file), and the writer's output is checked for the same fields,
enum tagging and byte encoding."""
import json
import struct

import numpy as np

from numrs_amd import checkpoint as ck


def _serde_like_doc():
    """What save_checkpoint(create_mlp(...), TrainingState::new_adam(1e-3)) writes
    for w1[2,3], b1[3] (ops/model.rs:150-176, 198-235; llo/model.rs:158-173, 238-252)."""
    w1 = np.arange(6, dtype=np.float32).reshape(2, 3) / 4
    b1 = np.array([0.5, -1.25, 3.0], np.float32)
    enc = lambda a: list(struct.pack("<%df" % a.size, *a.ravel()))  # noqa: E731
    return w1, b1, {
        "model": {
            "metadata": {"name": "training_model", "version": 1, "author": "NumRs",
                         "description": "Model created with NumRs", "domain": "ai.numrs",
                         "opset_version": 18, "producer_name": "NumRs",
                         "producer_version": "0.1.23", "metadata": {}},
            "graph": {"name": "training_model",
                      "nodes": [{"name": "fc1", "op_type": "Gemm", "inputs": ["input", "w1", "b1"],
                                 "outputs": ["hidden"], "attributes": {}}],
                      "inputs": [{"name": "input", "dtype": 1, "shape": [1, 2], "data": []}],
                      "outputs": ["hidden"],
                      "initializers": [{"name": "w1", "dtype": 1, "shape": [2, 3], "data": enc(w1)},
                                       {"name": "b1", "dtype": 1, "shape": [3], "data": enc(b1)}]}},
        "training_state": {"epoch": 3, "iteration": 300, "loss": 0.25,
                           "optimizer": {"Adam": {"learning_rate": 0.001, "beta1": 0.9,
                                                  "beta2": 0.999, "epsilon": 1e-08}},
                           "gradients": {}, "optimizer_state": {}}}


def test_reader_on_serde_layout(tmp_path):
    w1, b1, doc = _serde_like_doc()
    p = tmp_path / "ck.json"
    p.write_text(json.dumps(doc, indent=2))
    c = ck.load_checkpoint(str(p))
    assert c.name == "training_model" and c.epoch == 3 and c.iteration == 300
    assert c.loss == 0.25
    assert np.array_equal(c.initializers["w1"], w1) and np.array_equal(c.initializers["b1"], b1)
    assert c.optimizer == {"Adam": {"learning_rate": 0.001, "beta1": 0.9, "beta2": 0.999,
                                    "epsilon": 1e-08}}


class _FakeTensor:
    """values / gradient / device_ptrs, as checkpoint.save_checkpoint reads them."""

    def __init__(self, v, g, ptr):
        self.v, self.g, self.ptr = v, g, ptr

    def values(self):
        return self.v

    def gradient(self):
        return self.g

    def device_ptrs(self):
        return self.ptr, None


def test_writer_layout_matches_serde_fields(tmp_path):
    w = np.array([[1.5, -2.0], [np.float32(0.1), 7.0]], np.float32)
    g = np.array([[np.nan, 1.0], [2.0, np.inf]], np.float32)
    p = tmp_path / "out.json"
    ck.save_checkpoint(str(p), {"w": _FakeTensor(w, g, 1)}, None, epoch=2, iteration=5,
                       loss=0.5, name="m")
    doc = json.loads(p.read_text())
    assert set(doc) == {"model", "training_state"}
    assert set(doc["model"]) == {"metadata", "graph"}
    assert set(doc["model"]["metadata"]) == {"name", "version", "author", "description", "domain",
                                             "opset_version", "producer_name", "producer_version",
                                             "metadata"}
    assert set(doc["model"]["graph"]) == {"name", "nodes", "inputs", "outputs", "initializers"}
    init = doc["model"]["graph"]["initializers"][0]
    assert set(init) == {"name", "dtype", "shape", "data"}
    assert init["dtype"] == 1 and init["shape"] == [2, 2]
    assert bytes(init["data"]) == w.astype("<f4").tobytes()  # Vec<u8> as an array of numbers
    ts = doc["training_state"]
    assert set(ts) == {"epoch", "iteration", "loss", "optimizer", "gradients", "optimizer_state"}
    assert ts["optimizer"] == {"SGD": {"learning_rate": 0.0, "momentum": 0.0}}  # externally tagged
    assert ts["gradients"]["w"] == [None, 1.0, 2.0, None]  # serde_json writes non-finite f32 as null
    # f32 values survive the JSON round trip exactly
    c = ck.load_checkpoint(str(p))
    assert np.array_equal(c.initializers["w"], w)
    assert np.array_equal(c.gradients["w"][1:3], np.array([1.0, 2.0], np.float32))
