"""Writes lean_gpu_externs.txt: the @[extern] names the reference binds to GPU code.

Every extern of Puffer/Float/CUDA.lean (bodies in ffi/puffercuda.cu) and the externs of
Puffer/Float/BLAS.lean whose bodies in ffi/pufferblas.c use the GPU (cuBLAS / cuBLASLt / the CUDA
runtime, or another such entry). Reads the reference as text; run from the repository root:
    python tests/golden/make_lean_externs.py /root/reference
"""
import re
import sys
from pathlib import Path


def externs(lean_file):
    return re.findall(r'@\[extern "([A-Za-z0-9_]+)"\]', lean_file.read_text())


def c_body(src, name):
    m = re.search(r"LEAN_EXPORT[^;{]*\b" + name + r"\s*\(", src)
    if not m:
        return ""
    i = src.index("{", m.end())
    depth = 0
    for j in range(i, len(src)):
        depth += {"{": 1, "}": -1}.get(src[j], 0)
        if depth == 0:
            return src[i:j + 1]
    return src[i:]


def main(ref):
    ref = Path(ref)
    cuda = externs(ref / "Puffer/Float/CUDA.lean")
    blas = externs(ref / "Puffer/Float/BLAS.lean")
    src = (ref / "ffi/pufferblas.c").read_text()
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)  # comments mention GPU calls that code does not make
    src = re.sub(r"//[^\n]*", " ", src)
    gpu_words = re.compile(r"cuda|cublas|lt_layer|MlpPolicy|mlp_policy_load")
    # the LSTM entries stay CPU code: their only device use is the cuda_lstm_ppo_grad_batch link-time
    # hook (pufferblas.c:46-50), which the library defines and answers with "no device"
    gpu_blas = [n for n in blas if gpu_words.search(c_body(src, n).replace("cuda_lstm_ppo_grad_batch", ""))]
    names = sorted(set(cuda) | set(gpu_blas))
    out = Path(__file__).with_name("lean_gpu_externs.txt")
    out.write_text("\n".join(names) + "\n")
    print(f"{len(names)} names ({len(cuda)} from CUDA.lean, {len(gpu_blas)} GPU entries of BLAS.lean) -> {out}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
