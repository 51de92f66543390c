"""Write tests/golden/rocrand_uniform4.json from rocRAND's own device/host headers.

rocRAND (ROCm's open-source RNG library, /opt/rocm/include/rocrand) is what PyTorch-ROCm's
dropout draws through (curand_* -> hiprand_* -> rocrand_*). Its Philox4x32-10 engine and uniform
map are header-only `__device__ __host__` functions, so a host program compiled against them
gives their exact outputs on the CPU. The fixture pins oracle/philox.py's init layout (key,
counter words), draw order and uniform map.

Run in the build container (needs hipcc; no GPU): python tests/golden/make_rocrand_vectors.py
"""

import json
import os
import subprocess
import tempfile

CASES = [  # (seed, subsequence = thread, offset = 4 * ctr, number of uniform4 draws)
    (0, 0, 0, 3),
    (1234, 7, 40, 3),
    (20261031, 40959, 4 * 2016, 2),
    (2**63 + 12345, 524287, 4 * (2**32 - 1), 3),  # counter.x carries into counter.y
    (0xDEADBEEFCAFEF00D, 123456, 4 * 987654321, 2),
    (42, 2**32 - 1, 4 * 5, 2),
]

SRC = r"""
#include <rocrand/rocrand_kernel.h>
#include <cstdio>
#include <cstring>
static unsigned bits(float f) { unsigned u; std::memcpy(&u, &f, 4); return u; }
int main() {
  const unsigned long long cases[][4] = {%s};
  const int n = sizeof(cases) / sizeof(cases[0]);
  printf("[");
  for (int c = 0; c < n; ++c) {
    rocrand_state_philox4x32_10 a, b;
    rocrand_init(cases[c][0], cases[c][1], cases[c][2], &a);
    rocrand_init(cases[c][0], cases[c][1], cases[c][2], &b);
    printf("%%s{\"seed\": %%llu, \"subsequence\": %%llu, \"offset\": %%llu, \"draws\": [",
           c ? ", " : "", cases[c][0], cases[c][1], cases[c][2]);
    for (unsigned long long j = 0; j < cases[c][3]; ++j) {
      uint4 r = rocrand4(&a);
      float4 u = rocrand_uniform4(&b);
      printf("%%s{\"u32\": [%%u, %%u, %%u, %%u], \"f32_bits\": [%%u, %%u, %%u, %%u]}",
             j ? ", " : "", r.x, r.y, r.z, r.w, bits(u.x), bits(u.y), bits(u.z), bits(u.w));
    }
    printf("]}");
  }
  printf("]\n");
  return 0;
}
"""


def main():
    rows = ", ".join("{%dULL, %dULL, %dULL, %dULL}" % c for c in CASES)
    with tempfile.TemporaryDirectory() as tmp:
        src = os.path.join(tmp, "rr.cpp")
        exe = os.path.join(tmp, "rr")
        with open(src, "w") as f:
            f.write(SRC % rows)
        subprocess.run(["hipcc", "-O1", src, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    data = {"source": "rocRAND headers, ROCm " + _rocm_version(), "cases": json.loads(out)}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rocrand_uniform4.json")
    with open(path, "w") as f:
        json.dump(data, f, indent=1)
    print("wrote", path)


def _rocm_version():
    try:
        with open("/opt/rocm/.info/version") as f:
            return f.read().strip()
    except OSError:
        return "unknown"


if __name__ == "__main__":
    main()
