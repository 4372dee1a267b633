"""Compile the reference's CPU CSR->BCSR converter into oracle/_ref/.

Test infrastructure only.  The one source taken from the reference is
/root/reference/core/wrapper/convert_wrapper.cpp (plus the header it includes,
core/helper/macros.h), compiled where it lies; nothing is copied into this
repository.  The binding is oracle/ref_convert_bind.cpp.  The output is
oracle/_ref/ref_convert*.so, git-ignored, loaded by oracle.ref_csr_to_bcsr().
The reference's CUDA sources need nvcc and NVIDIA inline PTX and cannot be
built here.
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REF_SRC = "/root/reference/core/wrapper/convert_wrapper.cpp"


def build(verbose: bool = False) -> str:
    if not os.path.exists(REF_SRC):
        raise FileNotFoundError(REF_SRC)
    from torch.utils.cpp_extension import load
    out = os.path.join(HERE, "_ref")
    os.makedirs(out, exist_ok=True)
    load(name="ref_convert",
         sources=[REF_SRC, os.path.join(HERE, "ref_convert_bind.cpp")],
         build_directory=out,
         extra_cflags=["-O3", "-fopenmp", "-std=c++17"],
         extra_ldflags=["-fopenmp"],
         with_cuda=False,
         verbose=verbose)
    for f in os.listdir(out):
        if f.startswith("ref_convert") and f.endswith(".so"):
            return os.path.join(out, f)
    raise RuntimeError("reference converter build produced no .so")


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
