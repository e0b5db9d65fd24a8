"""Writes the golden fixtures under tests/golden/ (run in a checkout where the
reference is mounted; the tests only read what this script wrote).

compiler/  data files of the reference, copied unchanged (text) or gzipped
           (large CSVs): machine descriptions and register tables (inputs),
           a measured sweep (input), and what the reference's compiler
           produced from them (expected outputs):
             edge_<shape>_plans.csv     results/edge/<shape>/plans.csv
             predicted_full_rtx5060-laptop.csv.gz
                                        results/predicted_full_rtx5060-laptop.csv
             constants_rtx5060.cal      model/constants_rtx5060.cal
             calibrate_rtx5060.txt      results/calibrate_rtx5060.txt
           The shapes of the edge cases are restated in tests/test_compiler.py.
"""
import gzip
import os
import shutil
import sys

REF = os.environ.get("KVF_REFERENCE", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "compiler")

COPY = [
    ("machines/rtx5060-laptop.gpu", "rtx5060-laptop.gpu"),
    ("machines/rtx4060-laptop.gpu", "rtx4060-laptop.gpu"),
    ("machines/generic-gpu.gpu", "generic-gpu.gpu"),
    ("machines/resources_sm120.csv", "resources_sm120.csv"),
    ("machines/resources_sm89.csv", "resources_sm89.csv"),
    ("model/constants_rtx5060.cal", "constants_rtx5060.cal"),
    ("results/calibrate_rtx5060.txt", "calibrate_rtx5060.txt"),
]
EDGE = ["edge_g8_n3333", "edge_n129", "edge_odd_n", "edge_short"]
GZIP = [
    ("results/sweep_rtx5060-laptop.csv", "sweep_rtx5060-laptop.csv.gz"),
    ("results/predicted_full_rtx5060-laptop.csv", "predicted_full_rtx5060-laptop.csv.gz"),
]


def main():
    if not os.path.isdir(REF):
        sys.exit(f"reference checkout not found at {REF}")
    os.makedirs(OUT, exist_ok=True)
    for src, dst in COPY:
        shutil.copyfile(os.path.join(REF, src), os.path.join(OUT, dst))
    for e in EDGE:
        shutil.copyfile(os.path.join(REF, "results", "edge", e, "plans.csv"),
                        os.path.join(OUT, f"{e}_plans.csv"))
    for src, dst in GZIP:
        with open(os.path.join(REF, src), "rb") as f, \
                gzip.GzipFile(os.path.join(OUT, dst), "wb", compresslevel=9, mtime=0) as g:
            shutil.copyfileobj(f, g)
    print("wrote", len(os.listdir(OUT)), "files to", OUT)


if __name__ == "__main__":
    main()
