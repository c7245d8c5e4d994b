"""Applies the "Way 2" binding (pico's own GPU op seams calling libpico_amd.so)
to a COPY of pico's sources
(test infrastructure; the result is linked into oracle/_ref/libpico_way2.so by
oracle/Makefile's `way2` target, never into the product).

    python3 way2_patch.py <copy of the reference's src/>

It edits, in place, exactly these seams, by pattern:

* src/ops.c: pico_add / pico_sub / pico_mul replace their commented-out GPU
  stub (ops.c:42-44, 86-88, 130-132) with the GPU twin of libpico_amd.so, and
  pico_matmul gains the missing GPU branch (ops.c:178); a GPU output first
  gets device data and grad (pico_way2_adopt), and each op's _backward is the
  GPU hook for GPU tensors.
* src/tensor.c: pico_backward's seed (tensor.c:27-30) fills the entry grad
  with 1 on the device for a GPU entry.
* src/optim/SGD.c: the step and zero_grad loops (SGD.c:29-47) run pk_sgd_f32 /
  pk_fill_f32 for GPU params.
* src/arena.h: arena_reset and arena_destroy (arena.h:123-153) also rewind /
  release the arena's device blocks.

Every edit must apply exactly once, or the script fails.  No text of the
reference is stored here: the anchors are the few identifiers being wired.
"""
import os
import re
import sys

HEADER = """\
/* GPU seams of pico, bound to libpico_amd.so (its include/pico_amd.h) */
#pragma once
#include <stddef.h>
#include <stdint.h>
struct PicoTensor;
struct Arena;
int pico_add_gpu(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out);
int pico_sub_gpu(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out);
int pico_mul_gpu(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out);
int pico_matmul_gpu(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out);
void pico_add_backward_gpu(struct PicoTensor* self);
void pico_sub_backward_gpu(struct PicoTensor* self);
void pico_mul_backward_gpu(struct PicoTensor* self);
void pico_matmul_backward_gpu(struct PicoTensor* self);
void arena_device_reset(struct Arena* arena);
void arena_device_release(struct Arena* arena);
/* oracle/way2_glue.c */
int pico_way2_adopt(struct Arena* arena, struct PicoTensor* t);
void pico_way2_seed(struct PicoTensor* t);
void pico_way2_sgd(struct PicoTensor* t, float lr);
void pico_way2_zero_grad(struct PicoTensor* t);
"""


def edit(path, pattern, repl, count=1, flags=re.S):
    text = open(path).read()
    new, n = re.subn(pattern, repl, text, flags=flags)
    if n != count:
        sys.exit(f"way2_patch: {os.path.basename(path)}: pattern {pattern!r} matched {n} times, "
                 f"expected {count}")
    open(path, "w").write(new)


def function_edit(path, name, pattern, repl):
    """apply pattern -> repl once inside the body of function `name`"""
    text = open(path).read()
    m = re.search(r"\n[^\n]*\b" + re.escape(name) + r"\([^)]*\)\s*\{", text)
    if not m:
        sys.exit(f"way2_patch: {os.path.basename(path)}: function {name} not found")
    depth, i = 0, m.end() - 1
    while True:  # the matching closing brace of the body
        depth += {"{": 1, "}": -1}.get(text[i], 0)
        if depth == 0:
            break
        i += 1
    body = text[m.end():i]
    new, n = re.subn(pattern, repl, body, flags=re.S)
    if n != 1:
        sys.exit(f"way2_patch: {name}: pattern {pattern!r} matched {n} times, expected 1")
    open(path, "w").write(text[:m.end()] + new + text[i:])


def main(src):
    open(os.path.join(src, "pico_way2.h"), "w").write(HEADER)
    ops = os.path.join(src, "ops.c")
    edit(ops, r'(#include "tensor.h"\n)', r'\1#include "pico_way2.h"\n')
    for op in ("add", "sub", "mul"):
        # the stub comment (pico_mul's names pico_sub_gpu) becomes the twin call
        function_edit(ops, f"pico_{op}", r"//\s*pico_\w+_gpu\(a, b, out\);",
                      f"if(pico_way2_adopt(arena, out) || pico_{op}_gpu(a, b, out)) return NULL;")
        function_edit(ops, f"pico_{op}", rf"out->_backward = pico_{op}_backward;",
                      f"out->_backward = a->backend == GPU ? pico_{op}_backward_gpu : "
                      f"pico_{op}_backward;")
    function_edit(ops, "pico_matmul", r"(pico_matmul_cpu\(a, b, out\);\s*\})",
                  r"\1 else if(pico_way2_adopt(arena, out) || pico_matmul_gpu(a, b, out)) {"
                  r" return NULL; }")
    function_edit(ops, "pico_matmul", r"out->_backward = pico_matmul_backward;",
                  "out->_backward = a->backend == GPU ? pico_matmul_backward_gpu : "
                  "pico_matmul_backward;")

    tensor = os.path.join(src, "tensor.c")
    edit(tensor, r'(#include "ops.h"\n)', r'\1#include "pico_way2.h"\n')
    function_edit(tensor, "pico_backward",
                  r"(for\s*\(int i = 0; i < curr->numel; i\+\+\)\s*\{\s*curr->grad\[i\] = 1\.0f;\s*\})",
                  r"if(curr->backend == GPU) pico_way2_seed(curr); else \1")

    sgd = os.path.join(src, "optim", "SGD.c")
    edit(sgd, r'(#include "tensor.h"\n)', r'\1#include "pico_way2.h"\n')
    function_edit(sgd, "pico_optim_sgd_step", r"(tensor = optim->params\.data\[i\];)",
                  r"\1 if(tensor->backend == GPU) { pico_way2_sgd(tensor, optim->lr); continue; }")
    function_edit(sgd, "pico_optim_sgd_zero_grad", r"(tensor = optim->params\.data\[i\];)",
                  r"\1 if(tensor->backend == GPU) { pico_way2_zero_grad(tensor); continue; }")

    arena = os.path.join(src, "arena.h")
    edit(arena, r"(static inline void arena_reset\(struct Arena\* arena\) \{)",
         r"void arena_device_reset(struct Arena* arena);\n"
         r"void arena_device_release(struct Arena* arena);\n\1 arena_device_reset(arena);")
    edit(arena, r"(static inline void arena_destroy\(struct Arena\* arena\) \{)",
         r"\1 arena_device_release(arena);")


if __name__ == "__main__":
    if len(sys.argv) != 2 or not os.path.isdir(sys.argv[1]):
        sys.exit("usage: way2_patch.py <copy of the reference's src/>")
    main(sys.argv[1])
