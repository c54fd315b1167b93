"""Host bookkeeping of the layer kernel's call epochs (epoch_book.h),
compiled on its own with g++: epochs are never 0 (the device flags start
at 0) and each timed-out epoch is reported exactly once."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

DRIVER = r"""
#include <cstdio>
#include "epoch_book.h"
int main() {
  fdm::EpochBook b;
  int bad = 0;
  if (b.next() != 1u || b.next() != 2u) bad |= 1;
  b.epoch = 0xFFFFFFFFu;                      // wrap: skip 0
  if (b.next() != 1u) bad |= 2;
  fdm::EpochBook r;
  if (r.new_error(0)) bad |= 4;               // no wait gave up
  if (!r.new_error(7)) bad |= 8;              // epoch 7 timed out: reported
  if (r.new_error(7)) bad |= 16;              // ... once
  if (!r.new_error(9)) bad |= 32;             // a later call timed out too
  if (r.new_error(9) || r.new_error(0)) bad |= 64;
  std::printf("%d\n", bad);
  return bad != 0;
}
"""


def test_epoch_book(tmp_path):
    src = tmp_path / "epoch_book_test.cpp"
    exe = tmp_path / "epoch_book_test"
    src.write_text(DRIVER)
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "flash_deepseek_amd", "csrc"),
                    str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "0", out.stdout
