'use strict';
// ssm_ref.js -- single-threaded JavaScript restatement of the Mamba-2 SSD recurrence
// (TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg runs it as the reference's own
// execution model, plain JS on one host core; nothing in ssmjs_amd loads it).
//
// The reference runs its SSM arithmetic in MambaCode.js (absent: package-lock.json:1231-1241),
// either as WGSL on a WebGPU adapter or as a JS fallback on a CPU adapter
// (src/session/session.ts:127-128). This file restates the arithmetic of that fallback from the
// published algorithm (Dao & Gu 2024, section 6, recurrent form; the same recurrence as
// orc_ssd_sequential in ssm_oracle.c), in JS numbers (double) with Float32Array storage.
//
// usage: node ssm_ref.js <input.bin> <output.bin> B L H P N
//   input.bin: float32 little-endian x (B,L,H,P), dt (B,L,H), A (H), Bm (B,L,N), Cm (B,L,N),
//              D (H); one group; dt' = softplus(dt); zero initial state.
//   output.bin: float32 y (B,L,H,P). Prints {"seconds": s} (the recurrence only).
const fs = require('fs');

function softplus(x) { return x > 20 ? x : Math.log1p(Math.exp(x)); }

function ssd(x, dt, A, Bm, Cm, D, y, B, L, H, P, N) {
  const h = new Float64Array(P * N);
  for (let b = 0; b < B; b++) {
    for (let hh = 0; hh < H; hh++) {
      h.fill(0);
      for (let t = 0; t < L; t++) {
        const r = b * L + t;
        const delta = softplus(dt[r * H + hh]);
        const dA = Math.exp(delta * A[hh]);
        const xo = r * H * P + hh * P;
        const bo = r * N;
        for (let p = 0; p < P; p++) {
          const dx = delta * x[xo + p];
          const ho = p * N;
          let acc = 0;
          for (let n = 0; n < N; n++) {
            const v = dA * h[ho + n] + dx * Bm[bo + n];
            h[ho + n] = v;
            acc += v * Cm[bo + n];
          }
          y[xo + p] = acc + D[hh] * x[xo + p];
        }
      }
    }
  }
}

function main() {
  const [inp, outp, ...dims] = process.argv.slice(2);
  const [B, L, H, P, N] = dims.map(Number);
  const buf = fs.readFileSync(inp);
  const f = new Float32Array(buf.buffer, buf.byteOffset, buf.byteLength / 4);
  let o = 0;
  const take = (n) => { const a = f.subarray(o, o + n); o += n; return a; };
  const x = take(B * L * H * P);
  const dt = take(B * L * H);
  const A = take(H);
  const Bm = take(B * L * N);
  const Cm = take(B * L * N);
  const D = take(H);
  const y = new Float32Array(B * L * H * P);
  const t0 = process.hrtime();
  ssd(x, dt, A, Bm, Cm, D, y, B, L, H, P, N);
  const dtm = process.hrtime(t0);
  fs.writeFileSync(outp, Buffer.from(y.buffer));
  process.stdout.write(JSON.stringify({ seconds: dtm[0] + dtm[1] * 1e-9 }) + '\n');
}

main();
