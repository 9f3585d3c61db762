"""CPU test of how the executor maps the device's failure state to the reference's errors
(vortex-rt_amd/csrc/vrt_g3_errors.hpp; src/gemma3.cpp:1609-1696 and :1857-1863). The device keeps
the minimum code raised: block l's softmax failure is 2l and its non-finite hidden state 2l + 1,
so the error the reference would throw first wins; an abort word left raised by the persistent
kernel is always reported, even when a block's code hides the hand-off code."""
import os
import subprocess

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

OK, NUMERIC, HIP = 0, 4, 2
CASES = [
    ((0xFFFFFFFF, 0), (OK, "")),
    ((2 * 3 + 1, 0), (NUMERIC, "Non-finite value after Gemma 3 block 3")),
    ((1, 0), (NUMERIC, "Non-finite value after Gemma 3 block 0")),
    ((2 * 17 + 1, 0), (NUMERIC, "Non-finite value after Gemma 3 block 17")),
    ((2 * 5, 0), (NUMERIC, "Gemma 3 attention softmax failed")),
    ((0, 0), (NUMERIC, "Gemma 3 attention softmax failed")),
    ((0x20000000, 1), (HIP, "Gemma 3 decode: device hand-off timed out")),
    ((0x20000000, 0), (HIP, "Gemma 3 decode: device hand-off timed out")),
    ((0xFFFFFFFF, 1), (HIP, "Gemma 3 decode: device hand-off timed out")),
    ((2 * 7 + 1, 1), (NUMERIC, "Non-finite value after Gemma 3 block 7 (a device hand-off was also abandoned)")),
    ((2 * 2, 1), (NUMERIC, "Gemma 3 attention softmax failed (a device hand-off was also abandoned)")),
]


def test_failure_mapping(tmp_path):
    exe = str(tmp_path / "state_map_test")
    subprocess.run(["g++", "-O1", "-std=c++17", "-I" + os.path.join(REPO, "include"),
                    "-I" + os.path.join(REPO, "vortex-rt_amd", "csrc"), "-o", exe,
                    os.path.join(REPO, "tests", "cpp", "state_map_test.cpp")], check=True)
    inp = "".join(f"{nf:x} {ab:x}\n" for (nf, ab), _ in CASES)
    out = subprocess.run([exe], input=inp, capture_output=True, text=True, check=True).stdout.splitlines()
    assert len(out) == len(CASES)
    for line, (args, (code, msg)) in zip(out, CASES):
        c, m = line.split("|", 1)
        assert (int(c), m) == (code, msg), f"{args}: {line}"
