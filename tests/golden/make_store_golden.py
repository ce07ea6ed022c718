"""Write tests/golden/store_vectors.npz from the reference's store writer.

Run in the build container, where the reference checkout is mounted:

    python tests/golden/make_store_golden.py [/root/reference]

It compresses one seeded bf16 tensor with this package's encoder (whose bytes
equal the reference encoder's, pinned by codec_vectors.npz), then writes the
tensor's six arrays with the reference's own BinaryWeightWriter
(afterimage/runtime/binstore.py:50-77) in the order its store writer uses
(afterimage/runtime/streaming_engine.py:210-224, :362-365), recording the
resulting weights.bin bytes and each blob's reference (blobref_to_dict,
binstore.py:217-219). The file holds data only.
"""
from __future__ import annotations

import importlib.util
import json
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
OUT = HERE / "store_vectors.npz"
BLOBS = ("sign_mantissa", "packed", "chunk_offsets", "chunk_nbytes", "sym_lut", "len_lut")


def _reference_binstore(ref_root: Path):
    spec = importlib.util.spec_from_file_location(
        "reference_binstore", ref_root / "afterimage" / "runtime" / "binstore.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod  # dataclasses look the module up while it loads
    spec.loader.exec_module(mod)
    return mod


def main(ref_root: Path) -> None:
    sys.path.insert(0, str(ROOT))
    from afterimage_amd import workloads
    from afterimage_amd.runtime.compressed_store import compress_layer

    binstore = _reference_binstore(ref_root)
    w = workloads.bf16_normal((96, 1000), seed=11, scale=0.02, outlier_frac=1e-3)
    layer = compress_layer(w, chunk_size=1024, max_bits=12)
    enc = layer.encoded
    arrays = {"sign_mantissa": layer.sign_mantissa.numpy(), "packed": enc.packed,
              "chunk_offsets": enc.chunk_offsets, "chunk_nbytes": enc.chunk_nbytes,
              "sym_lut": enc.sym_lut, "len_lut": enc.len_lut}
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "weights.bin"
        with binstore.BinaryWeightWriter(path) as writer:
            blobs = {name: binstore.blobref_to_dict(writer.write(arrays[name])) for name in BLOBS}
        data = np.frombuffer(path.read_bytes(), dtype=np.uint8).copy()
    np.savez_compressed(OUT, weights_bin=data, blobs_json=np.array(json.dumps(blobs)),
                        bits=w.view(__import__("torch").int16).numpy().reshape(-1),
                        params=np.array([96, 1000, 1024, 12, 11], dtype=np.int64))
    print("wrote", OUT, data.nbytes, "bytes of weights.bin")


if __name__ == "__main__":
    main(Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference"))
