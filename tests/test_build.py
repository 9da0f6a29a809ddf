"""The build's source digests (kushkash_amd.build), which tie committed profiles to the code they
were measured on: comments and layout do not change a digest, code does."""
import importlib

build = importlib.import_module("kushkash_amd.build")


def test_code_drops_comments_and_layout_only():
    src = ('#define A 1 // one\n'
           '   int a = 1;   /* block\n  comment */  int b =  2;\n'
           '\n'
           'const char* s = "not // a comment /* either */";\n'
           "char q = '\"'; // a quote in a char literal\n")
    assert build._code(src) == ('#define A 1\n'
                                'int a = 1; int b = 2;\n'
                                'const char* s = "not // a comment /* either */";\n'
                                "char q = '\"';")


def test_comment_edits_keep_the_digest(tmp_path, monkeypatch):
    """A unit's digest over a copy of the sources: the same after a comment and indentation edit,
    different after a code edit."""
    csrc = tmp_path / "kushkash_amd" / "csrc"
    inc = tmp_path / "include"
    csrc.mkdir(parents=True)
    inc.mkdir()
    (csrc / "kush_common.h").write_text("#pragma once\nint f(int x) { return x + 1; }  // add one\n")
    (csrc / "unit.hip").write_text('#include "kush_common.h"\nint g() { return f(2); }\n')
    monkeypatch.setattr(build, "PKG", tmp_path / "kushkash_amd")
    monkeypatch.setattr(build, "ROOT", tmp_path)
    d0 = build.source_digest("unit.hip")
    (csrc / "kush_common.h").write_text("#pragma once\n// adds one\n    int f(int x) {  return x + 1; }\n")
    assert build.source_digest("unit.hip") == d0
    (csrc / "kush_common.h").write_text("#pragma once\nint f(int x) { return x + 2; }\n")
    assert build.source_digest("unit.hip") != d0
