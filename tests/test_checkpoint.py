"""Checkpoints on the CPU: SearchMamba.save_pretrained / from_pretrained
(engine/search_mamba.py's state_dict + JSON config) round-trip every tensor
bit for bit and the configuration, and loading never unpickles code
(torch.load with weights_only=True)."""

import json

import torch

from redpanda_amd.search_mamba import SearchMamba, SearchMambaConfig


def _model(seed):
    torch.manual_seed(seed)
    cfg = SearchMambaConfig(d_model=32, n_layer=2, d_state=12, n_track_state=4, mimo_p=2,
                            vocab_size=96)
    return SearchMamba(cfg, vocab_size=96, eval_dim=20)


def test_save_load_round_trip(tmp_path):
    m = _model(3)
    path = str(tmp_path / "search.pt")
    m.save_pretrained(path)
    cfg = json.load(open(SearchMamba._config_path(path)))
    assert cfg["eval_dim"] == 20 and cfg["d_state"] == 12 and cfg["n_track_state"] == 4
    back = SearchMamba.from_pretrained(path)
    a, b = m.state_dict(), back.state_dict()
    assert sorted(a) == sorted(b)
    for k in a:
        assert a[k].dtype == b[k].dtype and torch.equal(a[k], b[k]), k
    assert back.eval_dim == 20 and back.config == m.config


def test_load_is_weights_only(tmp_path, monkeypatch):
    m = _model(4)
    path = str(tmp_path / "search.pt")
    m.save_pretrained(path)
    seen = {}
    orig = torch.load

    def spy(*args, **kw):
        seen.update(kw)
        return orig(*args, **kw)

    monkeypatch.setattr(torch, "load", spy)
    SearchMamba.from_pretrained(path)
    assert seen.get("weights_only") is True
