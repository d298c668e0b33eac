"""The chat command line (cuqwen_amd/chat.py) without a GPU: usage and the
missing-file errors (no device work happens before the files are found)."""
import subprocess
import sys

import pytest

from cuqwen_amd import chat


def test_missing_files_are_reported(tmp_path, capsys):
    assert chat.main(["--weights", str(tmp_path / "none.bin"), "--tokenizer", str(tmp_path / "r.json")]) == 1
    assert "weight file" in capsys.readouterr().err
    w = tmp_path / "w.bin"
    w.write_bytes(b"\0" * 256)
    assert chat.main(["--weights", str(w), "--tokenizer", str(tmp_path / "r.json")]) == 1
    assert "tokenizer file" in capsys.readouterr().err


def test_weights_argument_is_required():
    r = subprocess.run([sys.executable, "-m", "cuqwen_amd.chat"], capture_output=True, text=True)
    assert r.returncode == 2 and "--weights" in r.stderr
