"""The C-ABI library (CPU side): exports, generator, tables, validation.

No compute call is made here: the engine's config validation runs before any
HIP call, so invalid configs are rejected on a machine without a GPU.
"""
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import MODEL_3B, ROOT, TINY

HEADER = os.path.join(ROOT, "include", "yuear.h")
LIB = os.path.join(ROOT, "yue2-mlx_amd", "libyuear.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(yuear_[a-z0-9_]+)\s*\(", text)) - {"yuear_token_callback"})


def test_library_exports_every_declared_symbol(yuear_lib):
    names = declared_functions()
    assert len(names) >= 25
    nm = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True,
                        check=True).stdout
    exported = set(re.findall(r"\bT (yuear_\w+)", nm))
    assert set(names) <= exported, set(names) - exported
    for name in names:  # resolvable through the loader as well
        assert getattr(yuear_lib.lib, name) is not None
    assert set(yuear_lib.EXPORTS) <= set(names)


def test_build_identifier(yuear_lib):
    assert yuear_lib.build_identifier().startswith("yuear-gfx950")


def test_tensor_ids_cover_every_reference_name(yuear_lib):
    shapes = yuear_lib.tensor_shapes(MODEL_3B)
    ids = [yuear_lib.lib.yuear_tensor_id(n.encode()) for n in shapes]
    assert min(ids) >= 0 and len(set(ids)) == len(ids) == 3 + 28 * 11
    for bad in (b"model.layers.x.mlp.up_proj.weight", b"lm_head", b"model.layers.0.mlp.weight"):
        assert yuear_lib.lib.yuear_tensor_id(bad) == -1


def test_generator_is_deterministic_and_normal(yuear_lib, oracle):
    a = yuear_lib.random_tensor("model.layers.0.mlp.up_proj.weight", (512, 512), seed=3)
    b = yuear_lib.random_tensor("model.layers.0.mlp.up_proj.weight", (512, 512), seed=3)
    c = yuear_lib.random_tensor("model.layers.0.mlp.gate_proj.weight", (512, 512), seed=3)
    np.testing.assert_array_equal(a, b)
    assert (a != c).mean() > 0.9
    x = oracle.bf16_to_f32(a).astype(np.float64)
    assert abs(x.mean()) < 1e-3 and abs(x.std() - 0.02) < 5e-4
    assert abs(np.mean(np.abs(x) < 0.02) - 0.6827) < 0.01  # one-sigma mass
    g = yuear_lib.random_tensor("model.norm.weight", (4096,), seed=3, norm_std=0.0)
    assert (g == 0x3F80).all()  # unit gains by default


def test_generator_matches_fixture_checksum(yuear_lib):
    g = np.load(os.path.join(ROOT, "tests", "golden", "tiny_model.npz"))
    w = yuear_lib.random_weights(TINY, int(g["seed"]), float(g["std"]), float(g["norm_std"]))
    total = np.uint64(0)
    for name in sorted(w):
        total += np.uint64(int(w[name].astype(np.uint64).sum()))
    assert total == g["weight_checksum"]


def test_rope_table_matches_oracle(yuear_lib, oracle):
    c1, s1 = yuear_lib.rope_table(3000, 128, 5e5)
    c2, s2 = oracle.rope_table(3000, 128, 5e5)
    np.testing.assert_array_equal(c1, c2)
    np.testing.assert_array_equal(s1, s2)
    assert (c1[0] == 0x3F80).all() and (s1[0] == 0).all()


@pytest.mark.parametrize("change,message", [
    (dict(num_key_value_heads=5), "divisible"),
    (dict(head_dim=64), "head_dim"),
    (dict(rms_norm_eps=0.0), "rms_norm_eps"),
    (dict(rope_theta=-1.0), "rope_theta"),
    (dict(hidden_size=100), "multiples of 64"),
    (dict(num_hidden_layers=0), "positive"),
])
def test_engine_rejects_invalid_configs_before_touching_the_gpu(yuear_lib, change, message):
    with pytest.raises(ValueError, match=message):
        yuear_lib.Engine(dict(TINY, **change))


def test_sampling_struct_defaults_follow_reference(yuear_lib):
    s = yuear_lib.sampling_struct(None)  # types.hpp:29-33
    assert (s.temperature, s.top_p, s.top_k, s.repetition_penalty, s.penalty_window,
            s.min_tokens, s.max_tokens) == (1.0, 0.95, 100, 1.2, 50, 200, 9000)


def test_cxx_facade_compiles_and_links(tmp_path):
    """include/yuear.hpp (the C++20 facade with the reference's
    generate_tokens signature) and its driver build against libyuear.so."""
    for name in ("facade_test", "pipeline_test"):
        out = tmp_path / name
        subprocess.run(["g++", "-std=c++20", "-O1", "-Wall", "-Wextra", "-Werror",
                        "-I" + os.path.join(ROOT, "include"),
                        os.path.join(ROOT, "tests", "cxx", name + ".cpp"), "-o", str(out),
                        "-L" + os.path.dirname(LIB), "-lyuear"], check=True)
        assert out.exists()


def test_cxx_facade_errors_keep_their_type(tmp_path, text_vocab):
    """Errors raised by library calls reach a C++ caller as yuear::Error with
    the library's type and message (host-only calls: no GPU needed)."""
    src = r'''
#include "yuear.hpp"
#include <cstdio>
template <class F> void expect(F f) {
  try { f(); std::printf("none\n"); }
  catch (const yuear::Error &e) { std::printf("%s: %s\n", e.type.c_str(), e.what()); }
}
int main(int, char **argv) {
  expect([] { yuear::Tokenizer t("/nonexistent/qwen.tiktoken"); });
  yuear::SongRequest r;
  r.style = "a";
  r.lyrics = "b";
  r.id = "../x";
  expect([&] { r.validate(); });
  const yuear::Tokenizer t(argv[1]);
  expect([&] { t.encode("ok\xff"); });
  r.id = "song";
  expect([&] { yuear::negative_prefix(r, t); });
  std::printf("%s|%d\n", t.decode(t.encode("Hello")).c_str(), int(yuear::token_prefixes(r, t).back()));
  const auto chunks = yuear::chunk_ranges(7, 10, 20);
  std::printf("%zu|%d|%d\n", chunks.size(), chunks.back().first, chunks.back().second);
  expect([] { yuear::chunk_ranges(0, 10); });
}
'''
    cpp, exe = tmp_path / "t.cpp", tmp_path / "t"
    cpp.write_text(src)
    subprocess.run(["g++", "-std=c++20", "-I" + os.path.join(ROOT, "include"), str(cpp), "-o",
                    str(exe), "-L" + os.path.dirname(LIB), "-lyuear",
                    "-Wl,-rpath," + os.path.dirname(LIB)], check=True)
    out = subprocess.run([str(exe), text_vocab[0]], capture_output=True, text=True,
                         check=True).stdout.splitlines()
    assert out[0].startswith("FileNotFoundError: /nonexistent/qwen.tiktoken")
    assert out[1] == "ValueError: id must be a filename-safe identifier"
    assert out[2] == "UnicodeDecodeError: Invalid UTF-8 text"
    assert out[3] == "ValueError: Symbolic CFG must retain the exact positive-branch ABC IDs"
    assert out[4] == "Hello|151847"
    assert out[5] == "3|6|7"
    assert out[6] == "ValueError: Empty codec or prefix leaves no acoustic context"


def test_cxx_facade_error_json_parser():
    """yuear::detail::json_string against the library's error JSON form."""
    src = r'''
#include "yuear.hpp"
#include <cstdio>
int main() {
  const std::string j = "{\"type\":\"ValueError\",\"message\":\"top_p must be in (0, 1] \\\"x\\\"\\n\"}";
  std::printf("%s|%s|", yuear::detail::json_string(j, "type").c_str(),
              yuear::detail::json_string(j, "message").c_str());
  std::printf("%d", int(yuear::detail::json_string(j, "missing").empty()));
}
'''
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        cpp, exe = os.path.join(d, "t.cpp"), os.path.join(d, "t")
        open(cpp, "w").write(src)
        subprocess.run(["g++", "-std=c++20", "-I" + os.path.join(ROOT, "include"), cpp, "-o", exe,
                        "-L" + os.path.dirname(LIB), "-lyuear",
                        "-Wl,-rpath," + os.path.dirname(LIB)], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    assert out == 'ValueError|top_p must be in (0, 1] "x"\n|1'
