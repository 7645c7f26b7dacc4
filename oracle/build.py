"""Build the C restatement of the oracle (``python -m oracle.build``).

TEST INFRASTRUCTURE ONLY: produces ``oracle/build/libavey_oracle.so`` from
``oracle/avey_oracle.c`` with gcc. The reference itself is Python and is never
built or run here.
"""

import os
import shutil
import subprocess

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(ORACLE_DIR, 'build')
LIB_PATH = os.path.join(OUT_DIR, 'libavey_oracle.so')


def build(verbose=True):
    os.makedirs(OUT_DIR, exist_ok=True)
    cc = shutil.which('gcc') or 'cc'
    src = os.path.join(ORACLE_DIR, 'avey_oracle.c')
    tmp = LIB_PATH + '.tmp'
    cmd = [cc, '-O2', '-fPIC', '-shared', '-std=c99', src, '-o', tmp, '-lm']
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'gcc failed:\n{res.stderr}')
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f'built {LIB_PATH}')
    return LIB_PATH


if __name__ == '__main__':
    build()
