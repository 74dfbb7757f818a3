"""Writes two GGUF fixtures with the reference's own tiny-model writer (tools/make_tiny_moe.py).

The reference's streaming test builds its model with `python3 -I tools/make_tiny_moe.py OUT`
(tools/test_streaming.sh:16); this script runs that same writer in a child process and keeps the bytes it
writes. The files are data: GGUF v3 models of random weights (F16 embedding, attention and router, F32
norms of 1.0, Q8_0 experts, Python's random.gauss with seed 1).
  * tiny_qwen3moe_reference.gguf: the writer's defaults (2 layers, n_embd 64, 2 query / 1 KV heads of 32,
    8 experts top-2 with f 32, vocab 256). tests/test_gguf_reference_file.py checks the reader against it.
  * tiny_qwen3moe_256_reference.gguf: the tiny model of the parity workload (2 layers, n_embd 256, 4 query /
    2 KV heads of 64, 8 experts top-2 with f 512, vocab 1024), written with the writer's own options
    --embd 256 --heads 4 --kv-heads 2 --ff-exp 512 --vocab 1024 (tools/make_tiny_moe.py:84-95).
    tests/test_gpu_reference_model.py runs the device path on it against the oracle and the reference's
    streaming identities (tools/test_streaming.sh:16-36).

    python3 tests/golden/make_tiny_gguf_fixture.py [/root/reference]
"""
import hashlib
import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = {
    "tiny_qwen3moe_reference.gguf": [],
    "tiny_qwen3moe_256_reference.gguf": ["--embd", "256", "--heads", "4", "--kv-heads", "2", "--ff-exp", "512",
                                         "--vocab", "1024"],
}


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    for name, args in FIXTURES.items():
        with tempfile.TemporaryDirectory() as tmp:
            path = os.path.join(tmp, "tiny.gguf")
            subprocess.run([sys.executable, "-I", os.path.join(ref, "tools/make_tiny_moe.py"), path] + args, check=True,
                           stdout=subprocess.DEVNULL)
            data = open(path, "rb").read()
        out = os.path.join(HERE, name)
        with open(out, "wb") as f:
            f.write(data)
        print(f"wrote {out}: {len(data)} bytes, sha256 {hashlib.sha256(data).hexdigest()}")


if __name__ == "__main__":
    main()
