"""Generate Philox4x32-10 known-answer vectors from rocRAND's open-source engine.

Compiles a tiny host program against /opt/rocm/include/rocrand/rocrand_philox4x32_10.h
(hipcc, host code only), runs it and writes philox_rocrand_kat.json next to this
script.  rocRAND's engine(seed, subsequence, offset) starts at counter
(offset/4, 0, subsequence_lo, subsequence_hi) with key (seed_lo, seed_hi), so each
vector is (counter, key) -> the four 32-bit outputs.
"""
import json
import subprocess
import tempfile
from pathlib import Path

SRC = r'''
#include <cstdio>
#include <rocrand/rocrand_philox4x32_10.h>
int main() {
    const unsigned long long seeds[] = {0ull, 1ull, 0xdeadbeefdeadbeefull, 0x123456789abcdef0ull, 0xffffffffffffffffull};
    const unsigned long long subs[] = {0ull, 1ull, 7ull, 0x300000005ull, 0xffffffff00000002ull};
    const unsigned long long offs[] = {0ull, 4ull, 4096ull * 4, 0xfffffff0ull * 4};
    for (auto s : seeds) for (auto q : subs) for (auto o : offs) {
        rocrand_device::philox4x32_10_engine e(s, q, o);
        const uint4 r = e.next4();
        std::printf("%llu %llu %llu %u %u %u %u\n", s, q, o, r.x, r.y, r.z, r.w);
    }
    return 0;
}
'''


def main():
    here = Path(__file__).resolve().parent
    with tempfile.TemporaryDirectory() as d:
        src = Path(d) / "kat.cpp"
        exe = Path(d) / "kat"
        src.write_text(SRC)
        subprocess.run(["hipcc", "-O1", "-x", "hip", "--offload-arch=gfx950", str(src), "-o", str(exe)],
                       check=True)
        out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    vectors = []
    for line in out.strip().splitlines():
        s, q, o, a, b, c, e = (int(t) for t in line.split())
        counter = [(o // 4) & 0xFFFFFFFF, (o // 4) >> 32, q & 0xFFFFFFFF, q >> 32]
        vectors.append({"seed": s, "subsequence": q, "offset": o, "counter": counter,
                        "key": [s & 0xFFFFFFFF, s >> 32], "out": [a, b, c, e]})
    (here / "philox_rocrand_kat.json").write_text(json.dumps(vectors, indent=0))
    print(f"wrote {len(vectors)} vectors")


if __name__ == "__main__":
    main()
