#!/bin/bash
# Host-side AddressSanitizer and UndefinedBehaviorSanitizer runs of the library's CPU code (no GPU needed):
# the GGUF reader on every fixture, each truncation of its first 64 KB and
# 20000 random header mutations (gguf_fuzz), and the host weight quantiser
# over every format, block counts 0-300 and larger, thread counts and special
# values (quant_fuzz); and ThreadSanitizer over the oracle's spinning pool
# (oracle_pool: 8-thread products and attention equal to 1-thread ones) and
# over the library's retired list and device-memory pool (pool_race: pushes
# and concurrent drains, every pointer back exactly once). The
# library's sanitizers instrument host code only (-Xarch_host);
# device code is built as usual. Usage, from the repository root:
#   bash tests/sanitize/run.sh
set -e
R=$(cd "$(dirname "$0")/../.." && pwd)
B=${TMPDIR:-/tmp}/tmh_sanitize; mkdir -p $B
F="--offload-arch=gfx950 -O1 -g -std=c++17 -fPIC -ffp-contract=off -fno-gpu-rdc -Xclang -target-feature -Xclang -packed-fp32-ops -Xarch_host -fsanitize=address,undefined -Xarch_host -fno-omit-frame-pointer -I $R/include"
pids=""
for f in tmh_runtime tmh_kernels tmh_decode tmh_llama tmh_gguf tmh_quant_host; do
  /opt/rocm/bin/hipcc $F -c $R/tensomite.cr_amd/csrc/$f.hip -o $B/$f.o > $B/$f.log 2>&1 &
  pids="$pids $!"
done
for d in gguf_fuzz quant_fuzz; do
  /opt/rocm/bin/hipcc -O1 -g -std=c++17 -Xarch_host -fsanitize=address,undefined -I $R/include -c $R/tests/sanitize/$d.cpp -o $B/$d.drv
done
for p in $pids; do wait $p; done
LIB="$B/tmh_runtime.o $B/tmh_kernels.o $B/tmh_decode.o $B/tmh_llama.o $B/tmh_gguf.o $B/tmh_quant_host.o"
for d in gguf_fuzz quant_fuzz; do
  /opt/rocm/bin/hipcc --offload-arch=gfx950 -fno-gpu-rdc -Xarch_host -fsanitize=address,undefined $LIB $B/$d.drv -o $B/$d
done
$B/gguf_fuzz $R/tests/golden/*/*.gguf
$B/quant_fuzz
gcc -O1 -g -std=c11 -ffp-contract=off -fsanitize=thread -pthread -march=x86-64 \
  $R/tests/sanitize/oracle_pool.c $R/oracle/tmq_oracle.c $R/oracle/tmq_llama.c -o $B/oracle_pool -lm
$B/oracle_pool
g++ -O1 -g -std=c++17 -fsanitize=thread -pthread $R/tests/sanitize/pool_race.cpp -o $B/pool_race
$B/pool_race 50000
