"""Regenerates rocrand_philox.json from rocRAND's host-callable Philox engine.

Run from the repository root: python tests/golden/make_rocrand_vectors.py
Needs hipcc (compiles rocrand_philox_vectors.cpp for the host only).
"""
import json
import pathlib
import subprocess
import tempfile

HERE = pathlib.Path(__file__).resolve().parent


def main() -> None:
    with tempfile.TemporaryDirectory() as tmp:
        exe = pathlib.Path(tmp) / "rocrand_vectors"
        subprocess.run(["hipcc", "-O1", "-o", str(exe), str(HERE / "rocrand_philox_vectors.cpp")], check=True)
        out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    data = json.loads(out)
    (HERE / "rocrand_philox.json").write_text(json.dumps(data, indent=1) + "\n")
    print(f"wrote {len(data)} cases")


if __name__ == "__main__":
    main()
