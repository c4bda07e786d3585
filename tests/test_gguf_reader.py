"""The binding's GGUF reader against the test writer (CPU only): the same
hyper-parameters as the reference's Engine::load would read
(qwen3moe.cpp:862-882) and the same tensor bytes."""
import numpy as np

import gguf_tools as gt


def test_read_gguf_round_trip(tmp_path, binding):
    spec = gt.test_tiny_spec()
    path = tmp_path / "tiny.gguf"
    gt.write_gguf(spec, str(path))
    kv, tensors = binding.read_gguf(str(path))
    assert kv["general.architecture"] == "qwen3moe"
    assert sorted(tensors) == sorted(spec.tensors)
    for name, (t, ne, data) in spec.tensors.items():
        rt, rne, rdata = tensors[name]
        assert rt == t and rne == list(ne), name
        assert np.array_equal(np.ascontiguousarray(rdata).view(np.uint8).reshape(-1),
                              np.ascontiguousarray(data).view(np.uint8).reshape(-1)), name
    hp = binding.gguf_hparams(kv, tensors, 1 << 20)
    for k in ("n_layer", "D", "n_head", "n_kv", "hd", "n_expert", "n_used", "FF", "n_vocab"):
        assert hp[k] == getattr(spec, k), k
    assert hp["n_ctx"] == spec.ctx_train  # min(ctx, context_length)
    assert abs(hp["eps"] - spec.eps) < 1e-12 and hp["rope_base"] == spec.rope_base
    assert binding.gguf_hparams(kv, tensors, 16)["n_ctx"] == 16


def test_read_gguf_rejects_other_files(tmp_path, binding):
    import pytest
    p = tmp_path / "x.bin"
    p.write_bytes(b"NOPE" + bytes(64))
    with pytest.raises(ValueError, match="not a GGUF"):
        binding.read_gguf(str(p))
