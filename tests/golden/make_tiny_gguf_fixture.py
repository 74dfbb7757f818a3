"""Writes tests/golden/tiny_qwen3moe_reference.gguf with the reference's own tiny-model writer.

The reference's streaming test builds its model with `python3 -I tools/make_tiny_moe.py OUT`
(tools/test_streaming.sh:16); this script runs that same command, with the writer's defaults (2 layers,
n_embd 64, 2 query / 1 KV heads of 32, 8 experts top-2 with f 32, vocab 256, seed 1: F16 embedding,
attention and router, F32 norms of 1.0, Q8_0 experts), in a child process, and keeps the bytes it writes
as a fixture. The file is data: a GGUF v3 model of random weights. tests/test_gguf_reference_file.py
checks the reader against it.

    python3 tests/golden/make_tiny_gguf_fixture.py [/root/reference]
"""
import hashlib
import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "tiny_qwen3moe_reference.gguf")


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "tiny.gguf")
        subprocess.run([sys.executable, "-I", os.path.join(ref, "tools/make_tiny_moe.py"), path], check=True,
                       stdout=subprocess.DEVNULL)
        data = open(path, "rb").read()
    with open(OUT, "wb") as f:
        f.write(data)
    print(f"wrote {OUT}: {len(data)} bytes, sha256 {hashlib.sha256(data).hexdigest()}")


if __name__ == "__main__":
    main()
