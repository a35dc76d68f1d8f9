"""Where the wide prefill GEMM's K steps go: barrier-arrival stamps.

  python -m surge_amd.gemm_stamps build OUTDIR [--prio]
      copies the package's sources (surge_amd/ and include/) to OUTDIR, adds
      s_memtime stamps to k_gemm_q8_wide (every wave of workgroup (0, 0)
      stamps the time right before each of its barriers over the 8-step turn
      that starts 64 K steps in; an exported sgk_gemm_stamps copies them
      out) and builds OUTDIR/surge_amd/libsurge_amd.so with the package
      Makefile; --prio also raises the staging waves' issue priority
      (s_setprio 3). Runs on the CPU: hipcc cross-compiles.
  python -m surge_amd.gemm_stamps run LIB
      on a GPU: with LIB (a stamped build) times the 27B shape's gate|up,
      down and DeltaNet input-projection products for a 512-token chunk
      (sg_gpu_time_gemm on layer 0 of a 4-layer synthetic model) and prints,
      per product, the duration of each step of the turn (last arrival to
      last arrival, s_memtime ticks) and the median time the consumer (MFMA)
      waves and the staging waves take from one barrier's last arrival to
      their own arrival at the next.

The product library is not changed: the stamps exist only in the copy.
"""
import argparse
import ctypes as C
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
WAVES, STEPS = 12, 8          # 8 consumer + 4 staging waves; one turn of 8 K steps


def _rep(src, old, new):
    if src.count(old) != 1:
        raise SystemExit(f"gemm_stamps: kernels.hip no longer has the expected text ({src.count(old)} matches): "
                         f"{old[:70]!r}")
    return src.replace(old, new)


def instrument(src, prio):
    """kernels.hip with the barrier stamps (and optionally the staging waves'
    priority) added to k_gemm_q8_wide."""
    src = _rep(src, 'template <int WT>\n__device__ __forceinline__ void gx_consume(',
               f'__device__ unsigned long long g_gstamp[{WAVES * STEPS}];\n'
               'extern "C" hipError_t sgk_gemm_stamps(void *h) {\n'
               '    return hipMemcpyFromSymbol(h, HIP_SYMBOL(g_gstamp), sizeof(g_gstamp), 0, hipMemcpyDeviceToHost);\n'
               '}\n'
               'template <int WT>\n__device__ __forceinline__ void gx_consume(')
    src = _rep(src, 'float (&wd)[2][GX_TM], uint32_t cb,\n'
                    '                                           uint32_t s, uint32_t kend, uint32_t wn, uint32_t wm, uint32_t li,\n'
                    '                                           uint32_t lg) {',
               'float (&wd)[2][GX_TM], uint32_t cb,\n'
               '                                           uint32_t s, uint32_t kend, uint32_t wn, uint32_t wm, uint32_t li,\n'
               '                                           uint32_t lg, bool rec, unsigned long long &ts) {')
    # the stamp's own wait (lgkmcnt(0)) comes before the barrier, where the
    # barrier's fence waits for the LDS anyway
    stamp = 'if (rec) { ts = __builtin_amdgcn_s_memtime(); __builtin_amdgcn_s_waitcnt(0xC07F); }'
    src = _rep(src, '                gm_tile_step(ac, ah, al, bh, dh);\n            }\n        }\n    }\n    __syncthreads();\n}',
               '                gm_tile_step(ac, ah, al, bh, dh);\n            }\n        }\n    }\n    ' + stamp
               + '\n    __syncthreads();\n}')
    rec = ('            const bool rec = s - kb0 == 64 && blockIdx.x == 0 && blockIdx.y == 0 && EPI != SGK_EPI_TILE;\n')
    save = ('        if (blockIdx.x == 0 && blockIdx.y == 0 && EPI != SGK_EPI_TILE && lane == 0)\n'
            '            for (int u = 0; u < 8; u++) g_gstamp[wave * 8 + u] = ts[u];\n')
    src = _rep(src, '        for (uint32_t s = kb0; s < kb1; s += 2 * NS) {\n#pragma unroll\n            for (int u = 0; u < 2 * NS; u++) {\n',
               '        unsigned long long ts[8] = {0, 0, 0, 0, 0, 0, 0, 0};\n'
               '        for (uint32_t s = kb0; s < kb1; s += 2 * NS) {\n' + rec
               + '#pragma unroll\n            for (int u = 0; u < 2 * NS; u++) {\n')
    src = _rep(src, '                __syncthreads();\n            }\n        }\n        return;',
               '                ' + stamp.replace('ts =', 'ts[u] =') + '\n                __syncthreads();\n'
               '            }\n        }\n' + save + '        return;')
    src = _rep(src, '    for (uint32_t s = kb0; s < kb1; s += 2 * NS) {\n#pragma unroll\n'
                    '        for (int u = 0; u < 2 * NS; u++) gx_consume<WT>(acc, xt, wq, wd, u & 1, s + u, kb1, wn, wm, li, lg);\n    }',
               '    unsigned long long ts[8] = {0, 0, 0, 0, 0, 0, 0, 0};\n'
               '    for (uint32_t s = kb0; s < kb1; s += 2 * NS) {\n' + rec.replace('            ', '        ', 1)
               + '#pragma unroll\n'
               '        for (int u = 0; u < 2 * NS; u++)\n'
               '            gx_consume<WT>(acc, xt, wq, wd, u & 1, s + u, kb1, wn, wm, li, lg, rec, ts[u]);\n    }\n'
               + save.replace('        ', '    ', 1).replace('\n            ', '\n        '))
    if prio:
        src = _rep(src, '    if (wave >= CW) {\n        const uint32_t pt = t - CW * 64;',
                   '    if (wave >= CW) {\n        __builtin_amdgcn_s_setprio(3);\n        const uint32_t pt = t - CW * 64;')
    return src


def build(out, prio):
    if os.path.exists(out):
        shutil.rmtree(out)
    ign = shutil.ignore_patterns("_build", "*.so", "__pycache__")
    shutil.copytree(HERE, os.path.join(out, "surge_amd"), ignore=ign)
    shutil.copytree(os.path.join(ROOT, "include"), os.path.join(out, "include"), ignore=ign)
    path = os.path.join(out, "surge_amd", "csrc", "kernels.hip")
    with open(path) as f:
        src = f.read()
    with open(path, "w") as f:
        f.write(instrument(src, prio))
    subprocess.run(["make", "-s", "-C", os.path.join(out, "surge_amd"), "-j8"], check=True)
    print(os.path.join(out, "surge_amd", "libsurge_amd.so"))


def run(lib_path):
    import numpy as np
    sys.path.insert(0, ROOT)
    import surge_amd as S
    S.LIB_PATH = os.path.abspath(lib_path)
    syn = S.Synth(dict(S.CFG_27B, n_layers=4), S.SG_T_Q8_0, seed=0)
    g = S.Gpu()
    g.load_model(syn.model)
    g.state_new(1024)
    read = S.lib().sgk_gemm_stamps
    read.argtypes = [C.c_void_p]
    read.restype = C.c_int
    for which, name in ((2, "gate|up 34816x5120"), (3, "down 5120x17408"), (0, "DeltaNet input projection 16480x5120")):
        us = g.time_gemm(0, which, 512, 5)
        buf = (C.c_uint64 * (WAVES * STEPS))()
        if read(buf):
            raise SystemExit("gemm_stamps: sgk_gemm_stamps failed")
        t = np.array(buf[:], dtype=np.int64).reshape(WAVES, STEPS)
        last = t.max(axis=0)
        cons = [int(np.median(t[:8, u] - last[u - 1])) for u in range(1, STEPS)]
        stag = [int(np.median(t[8:, u] - last[u - 1])) for u in range(1, STEPS)]
        print(f"{name}: {us:.1f} us per product (512 tokens)")
        print("  step duration (ticks):      ", np.diff(last).tolist())
        print("  consumer waves, release to arrival:", cons)
        print("  staging waves, release to arrival: ", stag)
    syn.close()


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    b = sub.add_parser("build")
    b.add_argument("out")
    b.add_argument("--prio", action="store_true")
    r = sub.add_parser("run")
    r.add_argument("lib")
    a = ap.parse_args()
    if a.cmd == "build":
        build(a.out, a.prio)
    else:
        run(a.lib)


if __name__ == "__main__":
    main()
