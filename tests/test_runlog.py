"""The ``training.riglog`` artefact (CPU): byte layout as documented in
``docs/RIGLOG_FORMAT.md:31-63``, the behaviour ``tests/test_logpack.py``
asks of the container, ``write_training_log`` (``rig/runlog.py:257-302``), and
the rest of a run directory: ``metrics.json``, the ``RIG_RESULT=`` line,
``validation.csv`` and ``checkpoint.npz`` (``rig/runlog.py:96-126,355-413``)."""

from __future__ import annotations

import csv
import dataclasses
import json
import math
import re
import struct

import numpy as np
import pytest

from gptrig import runlog


def _write(path, samples, columns=None, tokens_per_step=131_072, flops_per_token=1.5e9):
    with runlog.LogWriter(path, columns or runlog.training_columns(), tokens_per_step=tokens_per_step,
                          flops_per_token=flops_per_token) as writer:
        for step, values in samples:
            writer.append(step, values)


def test_bytes_follow_the_documented_offsets(tmp_path):
    # Built field by field from the layout table, not through the writer's own structs.
    columns = (runlog.Column(4), runlog.Column(7, 4, 2, -1, 1000), runlog.Column(9, 6, 1, 3, 8))
    path = tmp_path / "t.riglog"
    _write(path, [(3, (1.5, -2.0, 0.25)), (10, (0.0, 1e30, -1e-30))], columns, 4096, 2.5e8)
    raw = path.read_bytes()
    assert raw[0:8] == b"RIGLOG\x00\x01"
    assert int.from_bytes(raw[8:12], "little", signed=True) == 3
    assert raw[12:16] == b"\x00" * 4
    assert int.from_bytes(raw[16:24], "little", signed=True) == 4096
    assert struct.unpack("<d", raw[24:32])[0] == 2.5e8
    entry = raw[32 + 24:32 + 48]   # second column
    assert [int.from_bytes(entry[i:i + 4], "little", signed=True) for i in (0, 4, 8, 12)] == [7, 4, 2, -1]
    assert int.from_bytes(entry[16:24], "little", signed=True) == 1000
    third = raw[32 + 48:32 + 72]
    assert int.from_bytes(third[12:16], "little", signed=True) == 3
    start = 32 + 24 * 3
    assert start % 8 == 0
    assert int.from_bytes(raw[start:start + 4], "little", signed=True) == 3
    assert np.frombuffer(raw[start + 4:start + 16], "<f4").tolist() == [1.5, -2.0, 0.25]
    second = start + 16
    assert int.from_bytes(raw[second:second + 4], "little", signed=True) == 10
    assert np.frombuffer(raw[second + 4:second + 16], "<f4").tolist() == \
        np.array([0.0, 1e30, -1e-30], np.float32).tolist()
    assert len(raw) == second + 16


def test_reader_decodes_a_hand_built_file(tmp_path):
    raw = b"RIGLOG\x00\x01" + (2).to_bytes(4, "little") + b"\x00" * 4 + (1024).to_bytes(8, "little") \
        + struct.pack("<d", 3.0)
    raw += struct.pack("<iiiiq", 5, 1, -1, -1, 0) + struct.pack("<iiiiq", 6, 1, -1, -1, 0)
    raw += struct.pack("<iff", 1, 0.5, 2.0) + struct.pack("<iff", 2, 0.25, 4.0)
    path = tmp_path / "h.riglog"
    path.write_bytes(raw)
    log = runlog.read_log(path)
    assert [c.metric_id for c in log.columns] == [5, 6]
    assert log.tokens_per_step == 1024 and log.flops_per_token == 3.0
    np.testing.assert_array_equal(log.steps, [1, 2])
    np.testing.assert_array_equal(log.series("learning_rate"), [0.5, 0.25])
    np.testing.assert_array_equal(log.series("grad_norm"), [2.0, 4.0])
    assert log.series("train_loss") is None


def test_documented_measured_size():
    # 3,836 samples x 414 columns is the 6.38 MB diagnostics artefact of the format notes.
    total = runlog.header_size(414) + 3836 * runlog.record_size(414)
    assert total == 6_377_728
    assert round(total / 1e6, 2) == 6.38
    for n in range(1, 40):
        assert runlog.header_size(n) == 8 + 24 + 24 * n and runlog.header_size(n) % 8 == 0
        assert runlog.record_size(n) == 4 + 4 * n


def test_round_trip_preserves_float32_exactly(tmp_path):
    values = np.random.default_rng(7).standard_normal((64, 3), dtype=np.float32) * 1e6
    path = tmp_path / "t.riglog"
    _write(path, [(i + 1, row) for i, row in enumerate(values)])
    log = runlog.read_log(path)
    np.testing.assert_array_equal(log.values, values)
    np.testing.assert_array_equal(log.steps, np.arange(1, 65))
    assert path.stat().st_size == runlog.header_size(3) + 64 * runlog.record_size(3)


def test_derived_axes_stay_exact_beyond_float32(tmp_path):
    path = tmp_path / "t.riglog"
    _write(path, [(76_691, (2.88, 2.7e-4, 0.23))], tokens_per_step=131_072, flops_per_token=3.0644e9)
    log = runlog.read_log(path)
    tokens = log.axis("tokens_processed")
    assert tokens.dtype == np.int64 and int(tokens[0]) == 76_691 * 131_072
    flops = log.axis("cumulative_flops")
    exact = 76_691 * 131_072 * 3.0644e9
    assert flops.dtype == np.float64 and float(flops[0]) == exact
    assert float(np.float32(exact)) != exact
    np.testing.assert_array_equal(log.axis("step"), log.steps)
    with pytest.raises(KeyError):
        log.axis("train_loss")


def test_partial_trailing_record_is_dropped(tmp_path):
    path = tmp_path / "t.riglog"
    _write(path, [(s, (float(s), 0.0, 0.0)) for s in range(1, 11)])
    whole = path.read_bytes()
    for cut in range(1, runlog.record_size(3)):
        path.write_bytes(whole[:-cut])
        log = runlog.read_log(path)
        assert len(log.steps) == 9
        np.testing.assert_array_equal(log.steps, np.arange(1, 10))
    path.write_bytes(whole[:runlog.header_size(3)])
    assert runlog.read_log(path).values.shape == (0, 3)


def test_file_is_readable_after_every_append(tmp_path):
    path = tmp_path / "t.riglog"
    with runlog.LogWriter(path, runlog.training_columns(), tokens_per_step=8) as writer:
        for step in range(1, 6):
            writer.append(step, (float(step), 0.0, 0.0))
            log = runlog.read_log(path)
            assert len(log.steps) == step and float(log.series("train_loss")[-1]) == step


def test_steps_must_increase_and_widths_match(tmp_path):
    path = tmp_path / "t.riglog"
    with runlog.LogWriter(path, runlog.training_columns(), tokens_per_step=8) as writer:
        writer.append(5, (1.0, 2.0, 3.0))
        for bad in (5, 4):
            with pytest.raises(ValueError, match="must increase"):
                writer.append(bad, (1.0, 2.0, 3.0))
        with pytest.raises(ValueError, match="expected 3 values"):
            writer.append(6, (1.0, 2.0))


def test_foreign_and_truncated_files_are_refused(tmp_path):
    path = tmp_path / "t.riglog"
    for content, expected in ((b"", "bad magic"), (b"step,train_loss\n1,2.0\n", "bad magic"),
                              (runlog.MAGIC, "truncated inside its header"),
                              (runlog.MAGIC + b"\x00" * 8, "truncated inside its header"),
                              (runlog.MAGIC + struct.pack("<i4xqd", 0, 8, 1.0), "declares 0 columns"),
                              (runlog.MAGIC + struct.pack("<i4xqd", 2, 8, 1.0) + b"\x00" * 30,
                               "truncated inside its column table")):
        path.write_bytes(content)
        with pytest.raises(runlog.LogError, match=expected):
            runlog.read_log(path)


def test_header_rejects_impossible_configuration(tmp_path):
    path = tmp_path / "t.riglog"
    with pytest.raises(ValueError, match="tokens_per_step"):
        runlog.LogWriter(path, runlog.training_columns(), tokens_per_step=0)
    with pytest.raises(ValueError, match="flops_per_token"):
        runlog.LogWriter(path, runlog.training_columns(), tokens_per_step=8, flops_per_token=0.0)
    with pytest.raises(ValueError, match="at least one column"):
        runlog.LogWriter(path, [], tokens_per_step=8)


def test_registry_ids():
    # rig/metrics.py:81-86 and :136-140: ids are permanent.
    assert [runlog.METRIC_IDS[k] for k in ("step", "tokens_processed", "cumulative_flops", "train_loss",
                                           "learning_rate", "grad_norm")] == [1, 2, 3, 4, 5, 6]
    assert runlog.SCOPE_IDS["overall"] == 1 and runlog.SCOPE_IDS["block"] == 4
    assert [(c.metric_id, c.scope_id, c.layer, c.index, c.element_count)
            for c in runlog.training_columns()] == [(4, 1, -1, -1, 0), (5, 1, -1, -1, 0), (6, 1, -1, -1, 0)]


def test_write_training_log(tmp_path):
    # rig/runlog.py:257-302: the horizon-sized buffer is cut to final_step.
    horizon = np.zeros((8, 3), np.float32)
    horizon[:5] = np.random.default_rng(1).standard_normal((5, 3))
    path = runlog.write_training_log(tmp_path / "out", horizon, tokens_per_step=131_072, final_step=5)
    assert path.name == "training.riglog"
    assert not (tmp_path / "out" / ".training.riglog.tmp").exists()
    log = runlog.read_log(path)
    np.testing.assert_array_equal(log.steps, np.arange(1, 6))
    np.testing.assert_array_equal(log.values, horizon[:5])
    assert log.tokens_per_step == 131_072 and log.flops_per_token == 1.0
    np.testing.assert_array_equal(log.series("grad_norm"), horizon[:5, 2])

    again = runlog.write_training_log(tmp_path / "out", horizon[:2], tokens_per_step=64, final_step=2,
                                      flops_per_token=7.0)
    log = runlog.read_log(again)
    assert len(log.steps) == 2 and log.flops_per_token == 7.0 and log.tokens_per_step == 64

    with pytest.raises(ValueError, match="expected"):
        runlog.write_training_log(tmp_path, horizon[:3], tokens_per_step=8, final_step=4)
    with pytest.raises(ValueError, match="expected"):
        runlog.write_training_log(tmp_path, np.zeros((4, 2), np.float32), tokens_per_step=8, final_step=4)
    with pytest.raises(ValueError, match="flops_per_token"):
        runlog.write_training_log(tmp_path, horizon, tokens_per_step=8, final_step=4, flops_per_token=-1.0)


def test_reference_training_log_case(tmp_path):
    # tests/test_trainer_static.py:1055-1077 and :1111-1122 (early stop: a 5-row horizon, 2 steps taken).
    rows = np.asarray([[2.0, 1.0e-3, 0.5], [1.5, 5.0e-4, 0.25]], dtype=np.float32)
    horizon = np.zeros((5, 3), np.float32)
    horizon[:2] = rows
    for history in (rows, horizon):
        runlog.write_training_log(tmp_path, history, tokens_per_step=32, final_step=2, flops_per_token=10)
        log = runlog.read_log(tmp_path / runlog.TRAINING_LOG_NAME)
        assert [c.metric_id for c in log.columns] == [4, 5, 6]
        np.testing.assert_array_equal(log.steps, [1, 2])
        np.testing.assert_array_equal(log.values, rows)
        np.testing.assert_array_equal(log.axis("tokens_processed"), [32, 64])
        np.testing.assert_array_equal(log.axis("cumulative_flops"), [320.0, 640.0])


# --- metrics.json, RIG_RESULT=, validation.csv, checkpoint.npz ---------------------------------


def harness_accepts(payload, run_dir):
    """The acceptance rules of ``rig/harness/validation.py:301-387`` (no
    expected-token or checkpoint requirements), restated as a checker."""

    json.dumps(payload, allow_nan=False)
    assert payload.get("schema_version") == 1, "schema_version"
    assert payload.get("status") == "ok", "status"
    impl = payload.get("implementation")
    assert impl is None or isinstance(impl, dict), "implementation"
    metrics = payload.get("metrics")
    assert isinstance(metrics, dict), "metrics"
    t = metrics.get("train_seconds")
    assert isinstance(t, (int, float)) and not isinstance(t, bool) and math.isfinite(t) and t > 0, "train_seconds"
    n = metrics.get("tokens_processed")
    assert isinstance(n, int) and not isinstance(n, bool) and n > 0, "tokens_processed"
    loss = metrics.get("validation_loss")
    assert isinstance(loss, (int, float)) and not isinstance(loss, bool) and math.isfinite(loss) and loss >= 0, \
        "validation_loss"
    root = run_dir.resolve()
    declared = [payload["checkpoint"]] if payload.get("checkpoint") is not None else []
    artifacts = payload.get("artifacts", {})
    assert isinstance(artifacts, dict), "artifacts"
    for name, rel in artifacts.items():
        assert re.fullmatch(r"[A-Za-z0-9][A-Za-z0-9._-]{0,127}", name), "artifact name"
        declared.append(rel)
    for rel in declared:
        assert isinstance(rel, str) and rel.strip() and not rel.startswith("/"), "relative path"
        path = (root / rel).resolve()
        assert path.is_relative_to(root) and path.is_file(), f"contained file {rel}"
    return True



def _minimal_result(**metrics):
    return {"schema_version": 1, "status": "ok", "checkpoint": None,
            "artifacts": {"training_curve": "training.riglog"},
            "metrics": {"train_seconds": 1.5, "tokens_processed": 1024, "validation_loss": 3.25, **metrics}}


def test_harness_checker_refuses_what_the_harness_refuses(tmp_path):
    (tmp_path / "training.riglog").write_bytes(b"x")
    assert harness_accepts(_minimal_result(), tmp_path)
    bad = [dict(_minimal_result(), schema_version=2), dict(_minimal_result(), status="failed"),
           _minimal_result(train_seconds=0.0), _minimal_result(tokens_processed=0),
           _minimal_result(tokens_processed=True), _minimal_result(tokens_processed=10.0),
           _minimal_result(validation_loss=float("nan")), _minimal_result(validation_loss=-1.0),
           dict(_minimal_result(), artifacts={"training_curve": "../x"}),
           dict(_minimal_result(), artifacts={"training_curve": "/etc/passwd"}),
           dict(_minimal_result(), artifacts={"bad name": "training.riglog"}),
           dict(_minimal_result(), checkpoint="checkpoint.npz")]
    for payload in bad:
        with pytest.raises((AssertionError, ValueError)):
            harness_accepts(payload, tmp_path)


def test_write_result_and_result_line(tmp_path):
    result = _minimal_result(nested={"b": 2, "a": [1, 2.5]})
    path = runlog.write_result(tmp_path / "run", result)
    text = path.read_text()
    assert path.name == "metrics.json" and text.endswith("}\n")
    assert text == json.dumps(result, indent=2, sort_keys=True) + "\n"
    assert not (tmp_path / "run" / ".metrics.json.tmp").exists()
    line = runlog.result_line(result)
    assert line.startswith("RIG_RESULT=") and " " not in line and "\n" not in line
    assert json.loads(line[len("RIG_RESULT="):]) == result
    assert line.index('"a"') < line.index('"b"')  # sorted keys
    with pytest.raises(ValueError):
        runlog.write_result(tmp_path, _minimal_result(validation_loss=float("nan")))
    with pytest.raises(ValueError):
        runlog.result_line(_minimal_result(train_seconds=float("inf")))


def test_finite_metric():
    assert runlog.finite_metric("x", 0.0) == 0.0
    assert runlog.finite_metric("x", 2) == 2.0
    for value, positive in ((float("nan"), False), (float("inf"), False), (-1e-9, False), (0.0, True)):
        with pytest.raises(FloatingPointError, match="x must be finite"):
            runlog.finite_metric("x", value, positive=positive)


def test_write_validation_csv(tmp_path):
    rows = [runlog.ValidationRow(500, 65_536_000, "fineweb", "fineweb", 8192, 3.5, math.exp(3.5), 0.25, True),
            runlog.ValidationRow(500, 65_536_000, "downstream", "news", 4096, 4.0, math.exp(4.0), 0.125, False)]
    path = runlog.write_validation_csv(tmp_path, rows)
    with path.open(newline="") as handle:
        got = list(csv.reader(handle))
    assert got[0] == list(runlog.VALIDATION_CSV_HEADER)
    assert got[1] == ["500", "65536000", "fineweb", "fineweb", "8192", "3.5", repr(math.exp(3.5)), "0.25", "true"]
    assert got[2][2:4] == ["downstream", "news"] and got[2][-1] == "false"
    assert path.read_bytes().count(b"\r") == 0
    for bad in ([rows[1]], [rows[0], rows[0]], [dataclasses.replace(rows[0], kind="downstream")]):
        with pytest.raises(ValueError, match="one canonical"):
            runlog.write_validation_csv(tmp_path, bad)


def test_save_checkpoint(tmp_path):
    params = {"blocks/1/qkv_w": np.arange(6, dtype=np.float32).reshape(2, 3), "token_embedding": np.ones(4, np.float32),
              "blocks/0/qkv_w": np.zeros((2, 3), np.float32)}
    meta = {"seed": 3, "model": {"layers": 2}}
    path = runlog.save_checkpoint(tmp_path, params, meta)
    assert path.name == "checkpoint.npz" and not (tmp_path / ".checkpoint.npz.tmp").exists()
    with np.load(path, allow_pickle=False) as z:
        assert sorted(z.files) == ["metadata.json", "params/blocks/0/qkv_w", "params/blocks/1/qkv_w",
                                   "params/token_embedding"]
        np.testing.assert_array_equal(z["params/blocks/1/qkv_w"], params["blocks/1/qkv_w"])
        assert z["metadata.json"].dtype == np.uint8
        assert json.loads(z["metadata.json"].tobytes().decode()) == meta
        assert z["metadata.json"].tobytes().decode() == json.dumps(meta, sort_keys=True)


def test_run_driver_host_logic(capsys):
    pytest.importorskip("torch")
    from gptrig import run as grun
    from gptrig.train import GPTConfig

    import bench
    d = GPTConfig()
    assert grun.flops_per_token(d) * 131_072 == bench.step_flops(12, 768, 1024, 131_072, 50304)
    # Hand count for config D: 12 layers of 12 d^2 weights, the 50304-row head, causal QK^T/PV.
    assert grun.flops_per_token(d) == 3 * (2 * 12 * 768 * 768 * 12 + 2 * 768 * 50304 + 2 * 768 * 1025 * 12)
    cfg = grun.config_from_json('{"layers": 2, "optimizer": {"steps": 7, "warmup_steps": 1}}')
    assert cfg.layers == 2 and cfg.optimizer.steps == 7 and cfg.optimizer.warmup_steps == 1
    with pytest.raises(ValueError, match="unknown config fields"):
        grun.config_from_json('{"layer": 2}')
    # Refused before any device work: the reference's --stop-after-step past the schedule.
    assert grun.main(["--output-dir", "/nonexistent/x", "--config", '{"optimizer": {"steps": 3}}',
                      "--stop-after-step", "4"]) == 1
    assert "past the 3-step schedule" in capsys.readouterr().err
