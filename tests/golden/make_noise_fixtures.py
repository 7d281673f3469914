"""Copies the reference's Philox golden noise into tests/golden/m1_philox/.

Source: cuda_c_standalone/artifacts/m1_philox/{video,audio}_noise.bin of the
reference (raw little-endian bf16; recipe cuda_c_standalone/tests/m1_philox.cu:7-26
and tools/gen_ref.py:18-23: torch CUDA generator seeded 10, randn video
[1,3456,128] bf16 then audio [1,68,128] bf16 from the same generator, RTX 6000
Ada with 142 SMs).  The fixture manifest records shapes, the draw parameters
and SHA-256 of each payload.

Run from the repository root with the reference mounted at /root/reference.
"""
import hashlib
import json
import pathlib
import shutil

SRC = pathlib.Path("/root/reference/cuda_c_standalone/artifacts/m1_philox")
DST = pathlib.Path(__file__).resolve().parent / "m1_philox"

# Ada RTX 6000: 142 SMs, 1536 threads/SM -> grid cap 142*6 = 852 blocks of 256.
CASES = {
    "video_noise.bin": {"shape": [1, 3456, 128], "seed": 10, "offset": 0, "total_threads": 852 * 256},
    "audio_noise.bin": {"shape": [1, 68, 128], "seed": 10, "offset": 4, "total_threads": 34 * 256},
}


def main() -> None:
    DST.mkdir(parents=True, exist_ok=True)
    manifest = {}
    for name, meta in CASES.items():
        data = (SRC / name).read_bytes()
        shutil.copyfile(SRC / name, DST / name)
        manifest[name] = dict(meta, dtype="bfloat16", sha256=hashlib.sha256(data).hexdigest(), bytes=len(data))
    (DST / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print(json.dumps(manifest, indent=1))


if __name__ == "__main__":
    main()
