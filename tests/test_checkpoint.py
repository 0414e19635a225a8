"""The checkpoint files of the training loop (train.py:36-99), on the CPU.

* save_checkpoint / load_checkpoint round-trip the parameter tree exactly as
  nested dicts / lists of float32 NumPy arrays, the reference's layout.
* A plain pickle of such a tree (what the reference's pickle.dump of
  jax.device_get(params) writes) loads unchanged.
* Loading never runs code from the file: a pickle naming any global other
  than NumPy's array reconstructors is refused before anything is called.
* Files are written through a temporary name and renamed (no .tmp left).
"""
import os
import pickle

import numpy as np
import pytest
import torch

from nlearn_amd import checkpoint as ck
from nlearn_amd.model import BASELINE, init_params_numpy, tree_leaves


def test_roundtrip_and_layout(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    params_np = init_params_numpy(0, BASELINE)
    params = {"embeddings": {k: torch.from_numpy(v) for k, v in params_np["embeddings"].items()},
              "blocks": [{g: {k: torch.from_numpy(v) for k, v in d.items()} for g, d in b.items()}
                         for b in params_np["blocks"]],
              "ln_final": {k: torch.from_numpy(v) for k, v in params_np["ln_final"].items()},
              "lm_head": torch.from_numpy(params_np["lm_head"])}
    path = ck.save_checkpoint(params, 7, run_name="r")
    assert path == os.path.join("checkpoints", "r", "step_000007.pkl")
    assert sorted(os.listdir(os.path.join("checkpoints", "r"))) == ["step_000007.pkl"]
    back = ck.load_checkpoint(path)
    assert isinstance(back["blocks"], list) and isinstance(back["blocks"][0]["ffn"]["W1"], np.ndarray)
    for a, b in zip(tree_leaves(params_np), tree_leaves(back)):
        assert b.dtype == np.float32 and np.array_equal(a, b)


def test_plain_pickle_of_numpy_tree_loads(tmp_path):
    tree = {"a": {"w": np.arange(6, dtype=np.float32).reshape(2, 3)}, "b": [np.ones(4, np.float32)],
            "s": np.float32(2.5)}
    p = tmp_path / "ref.pkl"
    with open(p, "wb") as f:
        pickle.dump(tree, f)
    back = ck.load_checkpoint(str(p))
    assert np.array_equal(back["a"]["w"], tree["a"]["w"]) and np.array_equal(back["b"][0], tree["b"][0])
    assert back["s"] == np.float32(2.5)


def test_pickle_with_other_globals_is_refused(tmp_path):
    marker = tmp_path / "ran"
    # protocol-0 pickle that would call os.system("touch <marker>") if resolved
    payload = b"cos\nsystem\n(S'touch " + str(marker).encode() + b"'\ntR."
    p = tmp_path / "bad.pkl"
    p.write_bytes(payload)
    with pytest.raises(pickle.UnpicklingError, match="refusing"):
        ck.load_checkpoint(str(p))
    assert not marker.exists()
    # a tree containing a non-NumPy object is refused as well
    p2 = tmp_path / "obj.pkl"
    with open(p2, "wb") as f:
        pickle.dump({"x": torch.zeros(2)}, f)
    with pytest.raises(pickle.UnpicklingError):
        ck.load_checkpoint(str(p2))
