"""Writes philox_rocrand.json: Philox4x32-10 outputs computed by rocRAND's
header-only engine (an independent implementation shipped with ROCm), for
cross-checking the oracle's and the library's Philox beyond the published
Random123 vectors. Run: python tests/golden/make_philox_fixture.py
"""
import json
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = r'''
#include <cstdio>
#include <rocrand/rocrand_philox4x32_10.h>
struct Probe : rocrand_device::philox4x32_10_engine {
  uint4 run(uint4 c, uint2 k) { return ten_rounds(c, k); }
};
int main() {
  const unsigned v[][6] = {
    {0, 0, 0, 0, 0, 0}, {1, 0, 0, 0, 0, 0}, {0, 1, 0, 0, 0, 0}, {0, 0, 1, 0, 0, 0},
    {0, 0, 0, 1, 0, 0}, {0, 0, 0, 0, 1, 0}, {0, 0, 0, 0, 0, 1},
    {12345, 678, 0x59554541u, 0, 831001, 0}, {7, 3, 0x57454947u, 0, 1, 0},
    {0xdeadbeefu, 0xfeedfaceu, 0x01234567u, 0x89abcdefu, 0x13579bdfu, 0x2468ace0u}};
  Probe p;
  std::printf("[");
  for (unsigned i = 0; i < sizeof v / sizeof v[0]; ++i) {
    uint4 r = p.run(uint4{v[i][0], v[i][1], v[i][2], v[i][3]}, uint2{v[i][4], v[i][5]});
    std::printf("%s{\"ctr\":[%u,%u,%u,%u],\"key\":[%u,%u],\"out\":[%u,%u,%u,%u]}", i ? "," : "",
                v[i][0], v[i][1], v[i][2], v[i][3], v[i][4], v[i][5], r.x, r.y, r.z, r.w);
  }
  std::printf("]\n");
}
'''

if __name__ == "__main__":
    with tempfile.TemporaryDirectory() as tmp:
        src, exe = os.path.join(tmp, "p.cpp"), os.path.join(tmp, "p")
        open(src, "w").write(SRC)
        subprocess.run(["/opt/rocm/bin/hipcc", "-x", "hip", "--offload-arch=gfx950", src, "-o", exe],
                       check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    vectors = json.loads(out)
    json.dump(vectors, open(os.path.join(HERE, "philox_rocrand.json"), "w"), indent=0)
    print(len(vectors), "vectors")
