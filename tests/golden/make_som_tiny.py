"""Copies the reference's tiny converted model records (rootfs/models/tiny:
manifest.som and index.som, written by soso's own serializer; 2 KB of data)
into tests/golden/som_tiny/, where tests/test_som.py reads them.  The model's
shards are not copied: they predate the shard header and current soso refuses
them too (verify_shard, crates/sosomodel/src/index.rs:114-130).
Run: python tests/golden/make_som_tiny.py
"""
import os
import shutil

SRC = "/root/reference/rootfs/models/tiny"
DST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "som_tiny")

if __name__ == "__main__":
    os.makedirs(DST, exist_ok=True)
    for f in ("manifest.som", "index.som"):
        shutil.copyfile(os.path.join(SRC, f), os.path.join(DST, f))
        print("copied", f)
