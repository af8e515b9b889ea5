"""CPU checks of the ctd_generate protocol's request handling (include/ctd/generate.h;
reference tools/ctd_generate/main.cpp:36-64, 186-192): usage, and the error
reply for requests that fail before any device work.  The generation itself is
checked on the GPU (tests/test_gpu_infer.py) against oracle/generate.py.
"""
import json
import os
import subprocess

import pytest

from emberlm_amd import trainer as TR

EXE = os.path.join(os.path.dirname(TR.LIB_PATH), "ctd_generate")


def run(args, stdin=""):
    return subprocess.run([EXE, *args], input=stdin, capture_output=True, text=True, timeout=60)


def test_usage_without_model():
    r = run([])
    assert r.returncode == 2 and "usage:" in r.stderr and "--model" in r.stderr
    assert r.stdout == ""


@pytest.mark.parametrize("req,msg", [
    ('{"input_ids": [1, 2', "bad JSON"),
    ('[1, 2, 3]', "expected a JSON object"),
    ('{"max_new_tokens": 4}', "input_ids"),
    ('{"input_ids": "hello"}', "input_ids must be a list"),
    ('{"input_ids": [1, 2], "temperature": "hot"}', "temperature must be a number"),
    ('{"input_ids": [1, 2], "top_k": [3]}', "top_k must be an integer"),
    ('{"input_ids": [1, 2], "eos_ids": {"a": 1}}', "eos_ids must be a list"),
])
def test_bad_request_gives_error_line(req, msg):
    r = run(["--model", "/nonexistent/model.safetensors"], req)
    assert r.returncode == 1
    lines = r.stdout.splitlines()
    assert len(lines) == 1
    rec = json.loads(lines[0])
    assert list(rec) == ["done", "error", "reason"]          # nlohmann's sorted keys
    assert rec["done"] is True and rec["reason"] == "error" and msg in rec["error"]
    assert "ctd_generate: error:" in r.stderr


def test_missing_model_file_is_an_error_reply():
    r = run(["--model", "/nonexistent/model.safetensors"], '{"input_ids": [1, 2, 3]}')
    assert r.returncode == 1
    rec = json.loads(r.stdout)
    assert rec["reason"] == "error" and "cannot open" in rec["error"]
    assert "ctd_generate: weights /nonexistent/model.safetensors" in r.stderr


def test_error_text_is_escaped_json():
    r = run(["--model", "/x"], '{"input_ids": [1], "seed": "a\\"b\\n"}')
    rec = json.loads(r.stdout)            # parses: quotes and control characters escaped
    assert rec["reason"] == "error" and "seed" in rec["error"]
