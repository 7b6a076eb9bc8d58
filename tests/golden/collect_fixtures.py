"""Copy the hot-path conformance and network fixtures out of the reference.

Runs only in the build container, where the reference checkout is mounted.
It copies DATA (the `.tosa` graphs, `.npy` inputs/expected outputs and
`desc.json` metadata produced by ARM's TOSA reference model) into
`tests/golden/`; no reference source file is copied. The GPU box never needs
the reference: the tests read only the copies.

Usage: python tests/golden/collect_fixtures.py [/path/to/reference]
"""

import os
import shutil
import sys

# Operators whose conformance cases are kept: the hot path (CONV2D,
# DEPTHWISE_CONV2D, MATMUL, AVG_POOL2D, RESCALE), the glue a quantised CNN
# graph needs around it (CLAMP, ADD, RESHAPE, TRANSPOSE, CONST, CONST_SHAPE,
# IDENTITY), and the operators next to the path on the same GEMM and pooling
# cores (MATMUL_T, TRANSPOSE_CONV2D, CONV3D, MAX_POOL2D, CAST).
OPS = [
    "conv2d", "depthwise_conv2d", "matmul", "avg_pool2d", "rescale",
    "clamp", "add", "reshape", "transpose", "const", "const_shape", "identity",
    "matmul_t", "transpose_conv2d", "conv3d", "max_pool2d", "cast",
]


def main(ref):
    here = os.path.dirname(os.path.abspath(__file__))
    src_conf = os.path.join(ref, "tests", "conformance")
    dst_conf = os.path.join(here, "conformance")
    n = 0
    for op in OPS:
        for case in sorted(os.listdir(os.path.join(src_conf, op))):
            s = os.path.join(src_conf, op, case)
            if not os.path.isfile(os.path.join(s, "desc.json")):
                continue
            d = os.path.join(dst_conf, op, case)
            os.makedirs(d, exist_ok=True)
            for f in os.listdir(s):
                if f.endswith((".tosa", ".npy", ".json")):
                    shutil.copyfile(os.path.join(s, f), os.path.join(d, f))
            n += 1
    src_net = os.path.join(ref, "tests", "networks")
    dst_net = os.path.join(here, "networks")
    for case in sorted(os.listdir(src_net)):
        s = os.path.join(src_net, case)
        d = os.path.join(dst_net, case)
        os.makedirs(d, exist_ok=True)
        for f in os.listdir(s):
            if f.endswith((".tosa", ".npy", ".json")):
                shutil.copyfile(os.path.join(s, f), os.path.join(d, f))
        n += 1
    print(f"copied {n} cases")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
