"""Scratch-slot bookkeeping (csrc/slot_table.hpp) on the host: a slot grown after a graph capture keeps
the captured buffer alive (retired, not freed) until an explicit release."""
import os
import subprocess
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

DRIVER = textwrap.dedent(r"""
    #include <cstdio>
    #include <cstdlib>
    #include <set>
    #include "slot_table.hpp"
    static std::set<void*> live;
    static int fails = 0;
    #define CHECK(c) do { if (!(c)) { std::printf("FAIL line %d: %s\n", __LINE__, #c); fails++; } } while (0)
    int main() {
      ph::SlotTable<8> t;
      auto alloc = [](size_t n) -> void* { void* p = std::malloc(n); live.insert(p); return p; };
      auto fail_alloc = [](size_t) -> void* { return nullptr; };
      void* a = t.get(3, 1000, alloc);                 // first call of a shape
      CHECK(a && t.bytes[3] == 1024 && t.gen[3] == 1);
      void* captured = t.get(3, 1000, alloc);          // the call a graph captured
      CHECK(captured == a && t.gen[3] == 1 && t.retired.empty());
      void* b = t.get(3, 5000, alloc);                 // a larger call grows the slot
      CHECK(b && b != a && t.bytes[3] == 5120 && t.gen[3] == 2);
      CHECK(t.retired.size() == 1 && t.retired[0] == a && t.retired_bytes == 1024);
      CHECK(live.count(a) == 1);                       // the captured buffer is still allocated
      CHECK(t.get(3, 4000, alloc) == b);               // smaller requests reuse the grown buffer
      CHECK(t.get(3, 1 << 20, fail_alloc) == nullptr); // failed growth keeps the current buffer
      CHECK(t.peek(3) == b && t.bytes[3] == 5120);
      CHECK(t.get(9, 10, alloc) == nullptr && t.peek(-1) == nullptr);
      void* c = t.get(5, 0, alloc);                    // zero-byte requests get a real buffer
      CHECK(c && t.bytes[5] == 256);
      size_t n = t.release([](void* p) { live.erase(p); std::free(p); });
      CHECK(n == 1 && t.retired.empty() && t.retired_bytes == 0 && live.count(a) == 0);
      CHECK(live.count(b) == 1 && t.peek(3) == b);     // current buffers survive a release
      // a process whose shape grows step by step: every growth retires the previous buffer, all of
      // them stay allocated until a release, and a release frees exactly the retired ones
      size_t want = 5120, kept = 0;
      for (int i = 0; i < 10; i++) {
        kept += t.bytes[3];
        want += 4096;
        CHECK(t.get(3, want, alloc) != nullptr && t.bytes[3] >= want);
      }
      CHECK(t.retired.size() == 10 && t.retired_bytes == kept);
      CHECK(live.size() == 12);                        // 10 retired + slots 3 and 5 current
      CHECK(t.release([](void* p) { live.erase(p); std::free(p); }) == 10);
      CHECK(live.size() == 2 && t.retired.empty() && t.retired_bytes == 0);
      CHECK(t.get(3, want * 2, alloc) != nullptr && t.retired.size() == 1);  // the next growth retires one
      std::printf(fails ? "failed\n" : "ok\n");
      return fails ? 1 : 0;
    }
""")


def test_slot_table_retires_grown_buffers(tmp_path):
    src = tmp_path / "drv.cpp"
    src.write_text(DRIVER)
    exe = tmp_path / "drv"
    inc = os.path.join(ROOT, "pufferlean_amd", "csrc")
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", f"-I{inc}", str(src), "-o", str(exe)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        pytest.fail(r.stderr)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip().endswith("ok"), out.stdout + out.stderr
