"""Writes tests/golden/philox_rocrand.json: Philox4x32-10 outputs computed by
rocRAND's open-source engine (/opt/rocm/include/rocrand/rocrand_philox4x32_10.h,
host path), for counters/keys chosen to exercise carries and the key schedule.

Run in the build container: python tests/golden/make_philox_vectors.py
"""
import json
import subprocess
import tempfile
from pathlib import Path

CASES = [
    ([0, 0, 0, 0], [0, 0]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF, 0xFFFFFFFF]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0]),
    ([1, 0, 0, 0], [0, 0]),
    ([0, 0, 7, (3 << 8) | 1], [0, 0]),
    ([256, 0, 15, (16 << 8)], [12345, 0]),
    ([0xDEADBEEF, 0x1, 0x2, 0x3], [0x9E3779B9, 0xBB67AE85]),
]

SRC = r"""
#include <cstdio>
#include <rocrand/rocrand_philox4x32_10.h>
struct Probe : rocrand_device::philox4x32_10_engine {
    uint4 run(uint4 c, uint2 k) { return this->ten_rounds(c, k); }
};
int main() {
    unsigned v[6];
    Probe p;
    while (scanf("%u %u %u %u %u %u", &v[0], &v[1], &v[2], &v[3], &v[4], &v[5]) == 6) {
        uint4 c = make_uint4(v[0], v[1], v[2], v[3]);
        uint2 k = make_uint2(v[4], v[5]);
        uint4 o = p.run(c, k);
        printf("%u %u %u %u\n", o.x, o.y, o.z, o.w);
    }
}
"""


def main():
    with tempfile.TemporaryDirectory() as td:
        src = Path(td) / "probe.cpp"
        exe = Path(td) / "probe"
        src.write_text(SRC)
        subprocess.run(["hipcc", "-O1", "-x", "hip", "--offload-arch=gfx950", str(src), "-o", str(exe)],
                       check=True)
        inp = "\n".join(" ".join(str(x) for x in c + k) for c, k in CASES)
        out = subprocess.run([str(exe)], input=inp, capture_output=True, text=True, check=True).stdout
    rows = [list(map(int, line.split())) for line in out.strip().splitlines()]
    data = [dict(ctr=c, key=k, out=o) for (c, k), o in zip(CASES, rows)]
    path = Path(__file__).with_name("philox_rocrand.json")
    path.write_text(json.dumps(data, indent=1) + "\n")
    print(f"wrote {path} ({len(data)} vectors)")


if __name__ == "__main__":
    main()
