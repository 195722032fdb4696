"""Command line (inferencer-jetson_amd/__main__.py) on the CPU: the
reference's option checks (inferencer.cu:1604-1670), --help, and
--tokenize-only on a GGUF holding a Llama 3 shaped vocabulary (no GPU is
touched: the file is mapped and tokenized on the host)."""
import importlib.util
import io
import pathlib
import subprocess
import sys

import pytest

import gguf_writer as gw
import llama3_vocab as V
from conftest import ROOT, load_package

load_package()
import inferencer_jetson_amd.tokenizer as T  # noqa: E402

spec = importlib.util.spec_from_file_location("qk_cli", ROOT / "inferencer-jetson_amd" / "__main__.py")
cli = importlib.util.module_from_spec(spec)
spec.loader.exec_module(cli)


def run(args, stdin=""):
    out, err = io.BytesIO(), io.StringIO()
    rc = cli.run(args, stdout=out, stderr=err, stdin=io.StringIO(stdin))
    return rc, out.getvalue(), err.getvalue()


@pytest.fixture(scope="module")
def vocab_gguf(tmp_path_factory):
    pytest.importorskip("tokenizers")
    tokens, merges = V.trained_vocab(T.LLAMA3_SPLIT)
    w = gw.GGUFWriter()
    w.add("general.architecture", gw.STRING, "llama")
    w.add("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, list(tokens)))
    w.add("tokenizer.ggml.merges", gw.ARRAY, (gw.STRING, list(merges)))
    w.add_tensor("output_norm.weight", [256], 0, bytes(1024))   # a file holds tensor data
    path = tmp_path_factory.mktemp("cli") / "vocab.gguf"
    w.write(path)
    return path, T.Tokenizer([t.encode() for t in tokens], [m.encode() for m in merges])


def test_help():
    rc, out, _ = run(["--help"])
    assert rc == 0
    assert out.startswith(b"Usage:") and b"--prefill-batch N" in out and b"--compare-prefill" in out


@pytest.mark.parametrize("args,needle", [
    (["--bogus", "x"], "Unknown option: --bogus"),
    (["--max-tokens", "0", "x"], "positive --max-tokens"),
    (["--context", "64", "x"], "--context >= 128"),
    (["--gate-warps", "3", "x"], "must be 2, 4, 8, or 16"),
    (["--q6-warps", "32", "x"], "must be 2, 4, 8, or 16"),
    (["--prefill-batch", "33", "x"], "must be in 1..32"),
    (["--prefill-batch", "0", "x"], "must be in 1..32"),
    (["--prefill-batch", "4", "--float-q6", "x"], "one mode"),
    (["--compare-prefill", "x"], "requires --prefill-batch 2..32"),
    (["--compare-prefill", "--prefill-batch", "4", "--tokenize-only", "x"], "requires --prefill-batch 2..32"),
    (["--prompts-file", "/nonexistent/prompts.txt"], "Cannot open prompts file"),
    ([], "Provide prompts"),
])
def test_option_errors(args, needle):
    rc, out, err = run(args)
    assert rc == 1 and err.startswith("Error: ") and needle in err, err


def test_missing_model_is_an_error(tmp_path):
    rc, _, err = run(["--model", str(tmp_path / "none.gguf"), "--tokenize-only", "hi"])
    assert rc == 1 and err.startswith("Error: ")


def test_tokenize_only_prints_chat_prompt_ids(vocab_gguf, tmp_path):
    path, tok = vocab_gguf
    rc, out, err = run(["--model", str(path), "--tokenize-only", "hello world"])
    assert rc == 0
    # The load-time storage line: the file's one FP32 tensor of 256 values.
    assert err.startswith("Model: 0.000B parameters (FP32 100.0%), 32.00 bits per parameter") and \
        "Q4_K products in INT8, Q6_K products in INT8" in err, err
    want = T.chat_prompt(tok, "hello world")
    assert out == (" ".join(map(str, want)) + " \n").encode()
    # Several prompts from a file (CRLF lines, blank lines skipped): numbered.
    pf = tmp_path / "prompts.txt"
    pf.write_bytes("the matrix\r\n\r\nnaïve GPU\n".encode())
    rc, out, err = run(["--model", str(path), "--tokenize-only", "--prompts-file", str(pf)])
    assert rc == 0 and "Average over 2 prompts" in err
    lines = out.decode().splitlines()
    assert lines[0] == "[1/2] " + " ".join(map(str, T.chat_prompt(tok, "the matrix"))) + " "
    assert lines[1] == "[2/2] " + " ".join(map(str, T.chat_prompt(tok, "naïve GPU"))) + " "
    # The prompt from stdin when none is given.
    rc, out, _ = run(["--model", str(path), "--tokenize-only"], stdin="from stdin")
    assert rc == 0 and out == (" ".join(map(str, T.chat_prompt(tok, "from stdin"))) + " \n").encode()


def test_runs_as_a_directory_program(vocab_gguf):
    path, tok = vocab_gguf
    p = subprocess.run([sys.executable, str(ROOT / "inferencer-jetson_amd"), "--model", str(path), "--tokenize-only",
                        "x"], capture_output=True, timeout=120)
    assert p.returncode == 0, p.stderr.decode()[-2000:]
    assert p.stdout == (" ".join(map(str, T.chat_prompt(tok, "x"))) + " \n").encode()
