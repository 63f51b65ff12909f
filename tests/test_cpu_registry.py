"""Model description and registry preflight through the C ABI (host only: no GPU, no weights).

Reference: models::describe (src/models/mod.rs:32-64) and the preflight of Registry::load
(src/registry.rs:16-39): every file is opened and described and every name and alias checked before
any weights load, with these messages.
"""
import gguf_writer as gw
import pytest


def _meta_file(tmp_path, name, meta):
    path = str(tmp_path / name)
    open(path, "wb").write(gw.build(meta, []))
    return path


def test_describe_each_family(lh, tmp_path):
    ot = lh.describe(lh.Gguf.from_bytes(lh.SynthImage("openthai-tiny", seed=1)))
    assert ot == {"name": "openthai-systemone", "family": "openthai-systemone",
                  "architecture": "openthai_systemone", "aliases": [], "release_date": "2026-09-22"}
    la = lh.describe(lh.Gguf.from_bytes(lh.SynthImage("laya-tiny", seed=1)))
    assert la == {"name": "laya", "family": "english", "architecture": "ggmlc",
                  "aliases": ["english", "jev-latest"], "release_date": "2026-09-20"}
    for model, family in (("laya-multilingual", "multilingual"), ("laya-typed-decisions", "typed-decisions")):
        p = _meta_file(tmp_path, model + ".gguf", [("general.architecture", gw.STR, "ggmlc"),
                                                   ("laya.model_name", gw.STR, model)])
        d = lh.describe(lh.Gguf.open(p))
        assert (d["name"], d["family"], d["aliases"]) == (model, family, [family])
    # the laya-decoder family: named by general.name, no aliases
    dec = lh.describe(lh.Gguf.from_bytes(lh.SynthImage("tiny-q8", seed=1)))
    assert dec["name"] == "laya-decoder synthetic tiny-q8" and dec["family"] == "laya-decoder"
    assert dec["aliases"] == [] and dec["release_date"] == ""


def test_describe_rejects_other_models(lh, tmp_path):
    p = _meta_file(tmp_path, "kev.gguf", [("general.architecture", gw.STR, "ggmlc"),
                                          ("laya.model_name", gw.STR, "kev")])
    with pytest.raises(lh.LayaError, match="^unsupported ggmlc model kev$"):
        lh.describe(lh.Gguf.open(p))
    p = _meta_file(tmp_path, "llama.gguf", [("general.architecture", gw.STR, "llama")])
    with pytest.raises(lh.LayaError, match="^unsupported GGUF architecture llama$"):
        lh.describe(lh.Gguf.open(p))
    p = _meta_file(tmp_path, "none.gguf", [])
    with pytest.raises(lh.LayaError, match="^unsupported GGUF architecture $"):
        lh.describe(lh.Gguf.open(p))


def test_registry_preflight(lh, tmp_path):
    ot, la, dec = (str(tmp_path / n) for n in ("ot.gguf", "la.gguf", "dec.gguf"))
    lh.synth_file("openthai-tiny", 1, ot)
    lh.synth_file("laya-tiny", 1, la)
    lh.synth_file("tiny-q8", 1, dec)
    assert lh.registry_preflight([ot, la, dec]) == 0
    # names and aliases all select
    assert lh.registry_preflight([ot, la, dec], "jev-latest") == 1
    assert lh.registry_preflight([ot, la, dec], "english") == 1
    assert lh.registry_preflight([ot, la, dec], "laya-decoder synthetic tiny-q8") == 2
    with pytest.raises(lh.LayaError, match="^at least one model is required$"):
        lh.registry_preflight([])
    with pytest.raises(lh.LayaError, match="^duplicate model name or alias openthai-systemone; load one "
                                           "checkpoint per model$"):
        lh.registry_preflight([ot, dec, ot])
    with pytest.raises(lh.LayaError, match="^unknown default model nope$"):
        lh.registry_preflight([ot, la], "nope")
    # a file that does not open fails the whole preflight, wherever it sits in the list
    with pytest.raises(lh.LayaError):
        lh.registry_preflight([ot, str(tmp_path / "missing.gguf")])
    kev = _meta_file(tmp_path, "kev.gguf", [("general.architecture", gw.STR, "ggmlc"),
                                            ("laya.model_name", gw.STR, "kev")])
    with pytest.raises(lh.LayaError, match="^unsupported ggmlc model kev$"):
        lh.registry_preflight([ot, kev])
