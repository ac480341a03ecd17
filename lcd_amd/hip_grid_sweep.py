"""Grid sweep: the executor of axis stencils on a grid in natural order.

The DAG of a lower-triangular solve on a structured grid (every task waits
for its neighbours one step down along x, y and z) has ``nx + ny + nz - 2``
levels, and every persistent executor of this package pays at least one
polled hand-off per level.  The sweep removes the hand-off from all but the
faces between wavefronts:

* a LANE owns a grid line along x and runs its tasks one after the other:
  the value of the x neighbour is the register the lane wrote a step ago;
* a WAVEFRONT owns a bundle of ``WY x WZ`` lines (``WY * WZ = 64``, lane =
  ``ly + WY * lz``).  Lane (ly, lz) handles ``x = step - ly - SKZ * lz``, so
  the y neighbour's value is the lane below's register of the step before
  (one DPP row shift) and the z neighbour's value was written ``SKZ`` steps
  ago and comes through an LDS ring in the wavefront's own program order:
  nothing inside a bundle is polled;
* a WORKGROUP runs ``GY x GZ`` bundles.  A bundle's outer lines (a face) go
  to the neighbour bundle through LDS inside the workgroup and through a
  flagged buffer in memory between workgroups, the value being its own flag;
  helper wavefronts poll the memory faces and drop them into the same LDS
  arrays, so a sweeping wavefront only ever looks at LDS.

What a step needs besides the three values -- the coefficients of the
incoming entries by direction and the task's node loads (right-hand side,
diagonal, the prepared reciprocal of the diagonal) -- is laid out once per
set of values in the order the wavefronts consume it (``[bundle][step][pair]
[lane][2]``: three 16-byte loads per lane and step, fully coalesced), by two
generated staging kernels: one for what depends on the matrix arrays only
(run when their contents change), one for the rest (the right-hand side: run
in front of every solve).  The solution leaves in the same order and a third
kernel scatters it to the array.  The arithmetic of a task is the generated
text of the loop body, the sum in the order of the sequential loop (sources
ascending: z, y, x), the division ``lcd_div_checked``: the result is the
sequential loop's bit for bit.

Counterpart in the reference: none (its executors take one global task queue,
compiler/cuda_lowering.py:1343-1410); the role is that of its warp tasks.
"""

import ast
import re

from lcd_amd.hip_emitter import FLOAT, INT

SWEEP_DEPTH = 8                 # steps of operands a wavefront has in flight
SWEEP_TILE_STEPS = 32           # steps of a bundle one staging workgroup handles
SWEEP_MAX_LINE = 384            # longest grid line the LDS face arrays hold
SWEEP_ARGUMENTS = ("_lcd_sw_ops", "_lcd_sw_out", "_lcd_sw_yface",
                   "_lcd_sw_zface", "_lcd_sw_claim")
SWEEP_FLOAT_ARGUMENTS = SWEEP_ARGUMENTS[:4]
LDS_BYTES = 160 * 1024


def sweep_geometry(grid, wy=16, gy=1, gz=2, skz=2, components=6, dynamic=1):
    """Everything the kernels, the launcher and the runtime derive from the
    grid and the shape of the sweep (see the module text), as a dict."""
    nx, ny, nz = (int(extent) for extent in grid)
    wy, gy, gz, skz = int(wy), int(gy), int(gz), int(skz)
    if wy not in (8, 16) or gy < 1 or gz < 1 or skz not in (1, 2):
        raise ValueError("sweep shape: WY in (8, 16), GY, GZ >= 1, SKZ in (1, 2)")
    wz = 64 // wy
    nby, nbz = -(-ny // wy), -(-nz // wz)
    steps = nx + (wy - 1) + (wz - 1) * skz
    sp = -(-steps // SWEEP_DEPTH) * SWEEP_DEPTH
    ylag, zlag = wy - 1, (wz - 1) * skz
    # A step's record: the components the matrix gives, two to a plane of 64
    # lanes x 16 bytes (the last alone in a plane of 64 x 8 bytes when their
    # number is odd), then a plane of 64 x 8 bytes for every component that is
    # staged in front of each solve -- those are written as whole lines.
    static = int(components) - int(dynamic)
    pairs, halves = static // 2, static % 2 + int(dynamic)
    # (records per bundle: the loop's steps, the steps the prefetch runs
    # ahead, rounded up to the tiles of the staging kernels)
    spa = -(-(sp + SWEEP_DEPTH) // SWEEP_TILE_STEPS) * SWEEP_TILE_STEPS
    geometry = dict(
        nx=nx, ny=ny, nz=nz, wy=wy, wz=wz, gy=gy, gz=gz, skz=skz,
        nby=nby, nbz=nbz, bundles=nby * nbz, steps=steps, sp=sp,
        spa=spa, wgy=-(-nby // gy), wgz=-(-nbz // gz),
        waves=gy * gz, helpers=gy + gz, ylag=ylag, zlag=zlag,
        yrows=ylag + sp + 1, zrows=zlag + sp + 1, pairs=pairs,
        halves=halves, record=pairs * 128 + halves * 64,
        components=int(components))
    geometry["workgroups"] = geometry["wgy"] * geometry["wgz"]
    geometry["threads"] = (geometry["waves"] + geometry["helpers"]) * 64
    geometry["slots"] = geometry["bundles"] * geometry["spa"] * 64
    geometry["tiles"] = geometry["bundles"] * (spa // SWEEP_TILE_STEPS)
    geometry["lds_bytes"] = 8 * (
        geometry["waves"] * (geometry["yrows"] * wz + geometry["zrows"] * wy
                             + 8 * 64)
        + 2 * ((SWEEP_DEPTH + 1) * wy + 64)) + 64
    return geometry


def sweep_applies(grid, wy=16, gy=1, gz=2, skz=2):
    """True when the sweep serves this grid: three axes, lines the face
    arrays hold, and a workgroup that fits the LDS."""
    if grid is None or len(grid) != 3:
        return False
    nx, ny, nz = grid
    if nx < 2 or ny < 2 or nz < 2 or nx > SWEEP_MAX_LINE:
        return False
    return sweep_geometry(grid, wy, gy, gz, skz)["lds_bytes"] <= LDS_BYTES


_SWEEP_KERNEL = r"""
    // ---- grid sweep: a lane per grid line, a wavefront per bundle of lines
    constexpr int SW_NX = @nx@, SW_NY = @ny@, SW_NZ = @nz@, SW_WY = @wy@, SW_WZ = @wz@;
    constexpr int SW_GY = @gy@, SW_GZ = @gz@, SW_SKZ = @skz@, SW_D = @depth@;
    constexpr int SW_S = @steps@, SW_SP = @sp@, SW_SPA = @spa@, SW_P = @pairs@, SW_H8 = @halves@;
    constexpr int SW_NBY = @nby@, SW_NBZ = @nbz@, SW_WGY = @wgy@;
    constexpr int SW_NW = SW_GY * SW_GZ, SW_H = SW_GY + SW_GZ;
    constexpr int SW_YLAG = @ylag@, SW_ZLAG = @zlag@;
    constexpr int SW_YROWS = @yrows@, SW_ZROWS = @zrows@;
    constexpr int SW_YV = SW_S - SW_YLAG, SW_ZV = SW_S - SW_ZLAG;   // rows of a face that get written
    constexpr int SW_STEP_BYTES = SW_P * 1024 + SW_H8 * 512;
    static_assert(LCD_TPB == (SW_NW + SW_H) * 64, "workgroup size of the sweep");
    struct _s_shared_t {
        double yin[SW_NW][SW_YROWS][SW_WZ];     // incoming faces by the consumer's step (+ lag rows in front)
        double zin[SW_NW][SW_ZROWS][SW_WY];
        double ring[SW_NW][8][64];              // the wavefront's own values of the last steps
        double trash[(SW_D + 1) * SW_WY + 64];  // face writes of the lanes that have no face
        double zeros[(SW_D + 1) * SW_WY + 64];  // face reads of the lanes that have no face
        int slot;
    };
    __shared__ _s_shared_t _s_sh;
    const int _s_lane = threadIdx.x & 63;
    const int _s_wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const long long _lcd_t0 = (long long)wall_clock64();
    lcd_index_t _g_pos = 0, _g_src = 0; double _g_value = 0.0;
    double @operand@ = 0.0; double _lcd_wout = 0.0;
    (void)_g_pos; (void)_g_src; (void)_lane;
    auto _lcd_wdiv = [&](double a, double d, double r) { return lcd_div_checked_any(a, d, r); };
    (void)_lcd_wdiv;
    // the workgroups take their places in launch order: a place depends on
    // lower places only, and a place that is taken belongs to a workgroup
    // that runs, so the lowest unfinished one can always proceed
    if (threadIdx.x == 0) _s_sh.slot = atomicAdd(&_lcd_sw_claim[0], 1);
    __syncthreads();
    const int _s_place = _s_sh.slot;
    const int _s_wgy = _s_place % SW_WGY, _s_wgz = _s_place / SW_WGY;
    // the last wavefront of the launch leaves the counters as it found them
    auto _s_leave = [&]() {
        if (_s_lane == 0) {
            const int all = (int)gridDim.x * (LCD_TPB / 64);
            if (atomicAdd(&_lcd_sw_claim[1], 1) == all - 1) {
                __hip_atomic_store(&_lcd_sw_claim[1], 0, __ATOMIC_RELAXED, LCD_AGENT);
                __hip_atomic_store(&_lcd_sw_claim[0], 0, __ATOMIC_RELAXED, LCD_AGENT);
            }
        }
    };
    for (int c = threadIdx.x; c < SW_NW * SW_YROWS * SW_WZ; c += LCD_TPB) {
        const int w = c / (SW_YROWS * SW_WZ), s = (c / SW_WZ) % SW_YROWS - SW_YLAG;
        const int by = _s_wgy * SW_GY + w % SW_GY;
        (&_s_sh.yin[0][0][0])[c] = (by > 0 && s >= 0 && s < SW_YV) ? lcd_empty() : 0.0;
    }
    for (int c = threadIdx.x; c < SW_NW * SW_ZROWS * SW_WY; c += LCD_TPB) {
        const int w = c / (SW_ZROWS * SW_WY), s = (c / SW_WY) % SW_ZROWS - SW_ZLAG;
        const int bz = _s_wgz * SW_GZ + w / SW_GY;
        (&_s_sh.zin[0][0][0])[c] = (bz > 0 && s >= 0 && s < SW_ZV) ? lcd_empty() : 0.0;
    }
    for (int c = threadIdx.x; c < SW_NW * 8 * 64; c += LCD_TPB) (&_s_sh.ring[0][0][0])[c] = 0.0;
    for (int c = threadIdx.x; c < (SW_D + 1) * SW_WY + 64; c += LCD_TPB) { _s_sh.zeros[c] = 0.0; _s_sh.trash[c] = 0.0; }
    __syncthreads();
    if (_s_wave >= SW_NW) {
        // ---- helper: one face that comes from another workgroup, memory -> LDS
        __builtin_amdgcn_s_setprio(0);
        const int f = _s_wave - SW_NW;
        int w = 0, valid = 0, width = 1; double* src = nullptr; double* dst = nullptr;
        if (f < SW_GZ) {
            w = f * SW_GY; const int by = _s_wgy * SW_GY, bz = _s_wgz * SW_GZ + f;
            if (by > 0 && by < SW_NBY && bz < SW_NBZ) {
                valid = SW_YV; width = SW_WZ;
                src = _lcd_sw_yface + ((size_t)(by + SW_NBY * bz) * SW_YROWS + SW_YLAG) * SW_WZ;
                dst = &_s_sh.yin[w][SW_YLAG][0];
            }
        } else {
            w = f - SW_GZ; const int by = _s_wgy * SW_GY + w, bz = _s_wgz * SW_GZ;
            if (bz > 0 && by < SW_NBY && bz < SW_NBZ) {
                valid = SW_ZV; width = SW_WY;
                src = _lcd_sw_zface + ((size_t)(by + SW_NBY * bz) * SW_ZROWS + SW_ZLAG) * SW_WY;
                dst = &_s_sh.zin[w][SW_ZLAG][0];
            }
        }
        const int per = 64 / width;            // rows one load covers
        constexpr int K = 2;                   // loads in flight per poll
        const unsigned long long full = width == 64 ? ~0ull : ((1ull << width) - 1ull);
        int t = 0; unsigned spins = 0;
        while (t < valid) {
            double v[K]; bool mine[K];
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const int at = (t + k * per) * width + _s_lane;
                mine[k] = at < valid * width;
                v[k] = lcd_empty();
                if (mine[k]) v[k] = lcd_ld(&src[at]);
            }
            int rows = 0; bool open = true;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const unsigned long long m = __ballot(!mine[k] || !lcd_is_empty(v[k]));
                int r = 0;
                while (open && r < per && ((m >> (width * r)) & full) == full) ++r;
                if (open && mine[k] && _s_lane < r * width) {
                    const int at = (t + k * per) * width + _s_lane;
                    // into the workgroup's array; the slot in memory is empty again for
                    // the next launch
                    lcd_lds_st(&dst[at], v[k]); lcd_st(&src[at], lcd_empty());
                }
                if (open) rows += r;
                if (r < per) open = false;
            }
            t += rows;
            if (rows == 0) {
                __builtin_amdgcn_s_sleep(1);
                if ((++spins & 255u) == 0u && (lcd_gave_up((unsigned long long)spins << 4, _lcd_status, _lcd_t0)
                                               || lcd_load_relaxed(_lcd_status) != 0)) {
                    _lcd_status[0] = 1;
                    break;
                }
            }
        }
        _s_leave();
        return;
    }
    // ---- a sweeping wavefront
    const int _s_gy = _s_wave % SW_GY, _s_gz = _s_wave / SW_GY;
    const int _s_by = _s_wgy * SW_GY + _s_gy, _s_bz = _s_wgz * SW_GZ + _s_gz;
    if (_s_by >= SW_NBY || _s_bz >= SW_NBZ) { _s_leave(); return; }
    __builtin_amdgcn_s_setprio(3);
    auto _s_sweep = [&](auto _s_yg, auto _s_zg) {
        constexpr bool YG = decltype(_s_yg)::value, ZG = decltype(_s_zg)::value;
        const int beta = _s_by + SW_NBY * _s_bz;
        const int ly = _s_lane % SW_WY, lz = _s_lane / SW_WY;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(_lcd_sw_ops + (size_t)beta * SW_SPA * (SW_STEP_BYTES / 8)), 0, SW_SPA * SW_STEP_BYTES, 0x00020000);
        const unsigned loff = _s_lane * 16u, hoff = SW_P * 1024u + _s_lane * 8u;
        char* outp = (char*)(_lcd_sw_out + (size_t)beta * SW_SPA * 64) + _s_lane * 8u;
        lcd_v4u _s_o[SW_D][SW_P > 0 ? SW_P : 1];
        lcd_v2u _s_h[SW_D][SW_H8 > 0 ? SW_H8 : 1];
#pragma unroll
        for (int j = 0; j < SW_D; ++j) {
#pragma unroll
            for (int k = 0; k < SW_P; ++k)
                _s_o[j][k] = __builtin_amdgcn_raw_buffer_load_b128(rs, loff + k * 1024, j * SW_STEP_BYTES, 0);
#pragma unroll
            for (int k = 0; k < SW_H8; ++k)
                _s_h[j][k] = __builtin_amdgcn_raw_buffer_load_b64(rs, hoff + k * 512, j * SW_STEP_BYTES, 0);
        }
        const bool y_in_group = _s_gy + 1 < SW_GY, z_in_group = _s_gz + 1 < SW_GZ;
        // face writes inside the workgroup go to the consumer's array at
        // (own step - lag); every other lane writes the trash
        const bool yw_real = ly == SW_WY - 1 && _s_by + 1 < SW_NBY && y_in_group;
        const bool zw_real = lz == SW_WZ - 1 && _s_bz + 1 < SW_NBZ && z_in_group;
        double* yw = yw_real ? &_s_sh.yin[(_s_wave + 1) % SW_NW][0][lz] : &_s_sh.trash[_s_lane];
        double* zw = zw_real ? &_s_sh.zin[(_s_wave + SW_GY) % SW_NW][0][ly] : &_s_sh.trash[_s_lane];
        const int yw_inc = yw_real ? SW_D * SW_WZ : 0, zw_inc = zw_real ? SW_D * SW_WY : 0;
        // faces for other workgroups: one store of the whole wavefront through a
        // buffer descriptor of the consumer's array; the lanes that are not on the
        // face carry an offset beyond the array, which the hardware drops (no
        // change of the execution mask around the store)
        const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(_lcd_sw_yface + (size_t)(YG ? beta + 1 : beta) * SW_YROWS * SW_WZ), 0, SW_YROWS * SW_WZ * 8, 0x00020000);
        const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(_lcd_sw_zface + (size_t)(ZG ? beta + SW_NBY : beta) * SW_ZROWS * SW_WY), 0, SW_ZROWS * SW_WY * 8, 0x00020000);
        const unsigned yvo = ly == SW_WY - 1 ? lz * 8u : 0x80000000u;
        const unsigned zvo = lz == SW_WZ - 1 ? ly * 8u : 0x80000000u;
        // reads: the y face (first lanes of the rows; the others read zeros), the z
        // value from the face (first z row) or the ring (the row below)
        const double* yr = ly == 0 ? &_s_sh.yin[_s_wave][SW_YLAG][lz] : &_s_sh.zeros[_s_lane];
        const double* zf = lz == 0 ? &_s_sh.zin[_s_wave][SW_ZLAG][ly] : &_s_sh.zeros[_s_lane];
        const int yr_inc = ly == 0 ? SW_D * SW_WZ : 0, zf_inc = lz == 0 ? SW_D * SW_WY : 0;
        const double* zr = &_s_sh.ring[_s_wave][0][(_s_lane - SW_WY) & 63];
        double* rw = &_s_sh.ring[_s_wave][0][_s_lane];
        double _s_prev = 0.0;
        double fy = lcd_lds_ld(yr), vzf = lcd_lds_ld(zf), vzr = 0.0;
        unsigned spins = 0; bool dead = false;
        int soff = SW_D * SW_STEP_BYTES, ysoff = 0, zsoff = 0;     // (running offsets: no multiply per step)
        for (int s0 = 0; s0 < SW_SP; s0 += SW_D) {
#pragma unroll
            for (int j = 0; j < SW_D; ++j) {
                // (one wait for the step's records: the last of them is asked for first)
                if (SW_H8 > 0) asm volatile("" :: "v"(_s_h[j][SW_H8 > 0 ? SW_H8 - 1 : 0]));
                else asm volatile("" :: "v"(_s_o[j][SW_P > 0 ? SW_P - 1 : 0]));
@take@
                if (__builtin_expect(__ballot(!(fy == fy) || !(vzf == vzf)) != 0ull, 0)) {
                    // a value that is no number: the empty marker is waited for
                    while (!dead && __ballot(lcd_is_empty(fy) || lcd_is_empty(vzf)) != 0ull) {
                        fy = lcd_lds_ld(yr + j * SW_WZ);
                        vzf = lcd_lds_ld(zf + j * SW_WY);
                        if ((++spins & 1023u) == 0u && (lcd_gave_up(spins, _lcd_status, _lcd_t0)
                                                        || lcd_load_relaxed(_lcd_status) != 0))
                            dead = true;
                    }
                }
                const double _s_vz = lz == 0 ? vzf : vzr;
                const double fy_now = fy;
                // the faces of the next step and the z value of the row below, a step ahead
                fy = lcd_lds_ld(yr + (j + 1) * SW_WZ);
                vzf = lcd_lds_ld(zf + (j + 1) * SW_WY);
                if (SW_SKZ >= 2) vzr = lcd_lds_ld(zr + ((j + 1 - SW_SKZ) & 7) * 64);
@vy@
@task@
                _s_prev = _lcd_wout;
                lcd_lds_st(rw + (j & 7) * 64, _s_prev);
                if (SW_GY > 1) lcd_lds_st(yw + j * SW_WZ, _s_prev);
                if (SW_GZ > 1) lcd_lds_st(zw + j * SW_WY, _s_prev);
                if (YG) lcd_buffer_st(ry, yvo + j * (SW_WZ * 8), ysoff, _s_prev);
                if (ZG) lcd_buffer_st(rz, zvo + j * (SW_WY * 8), zsoff, _s_prev);
                *(double*)(outp + j * 512) = _s_prev;
#pragma unroll
                for (int k = 0; k < SW_P; ++k)
                    _s_o[j][k] = __builtin_amdgcn_raw_buffer_load_b128(rs, loff + k * 1024, soff + j * SW_STEP_BYTES, 0);
#pragma unroll
                for (int k = 0; k < SW_H8; ++k)
                    _s_h[j][k] = __builtin_amdgcn_raw_buffer_load_b64(rs, hoff + k * 512, soff + j * SW_STEP_BYTES, 0);
                if (SW_SKZ < 2) vzr = lcd_lds_ld(zr + ((j + 1 - SW_SKZ) & 7) * 64);
            }
            yr += yr_inc; zf += zf_inc; yw += yw_inc; zw += zw_inc;
            outp += SW_D * 512;
            soff += SW_D * SW_STEP_BYTES; ysoff += SW_D * SW_WZ * 8; zsoff += SW_D * SW_WY * 8;
        }
        if (dead) _lcd_status[0] = 1;
    };
    const bool _s_yglob = _s_by + 1 < SW_NBY && _s_gy + 1 == SW_GY;
    const bool _s_zglob = _s_bz + 1 < SW_NBZ && _s_gz + 1 == SW_GZ;
    if (_s_yglob) {
        if (_s_zglob) _s_sweep(lcd_flag<true>{}, lcd_flag<true>{}); else _s_sweep(lcd_flag<true>{}, lcd_flag<false>{});
    } else {
        if (_s_zglob) _s_sweep(lcd_flag<false>{}, lcd_flag<true>{}); else _s_sweep(lcd_flag<false>{}, lcd_flag<false>{});
    }
    _s_leave();
"""


_SWEEP_SLOT = r"""
    constexpr int SW_NX = @nx@, SW_NY = @ny@, SW_NZ = @nz@, SW_WY = @wy@, SW_WZ = @wz@;
    constexpr int SW_SKZ = @skz@, SW_SPA = @spa@, SW_P = @pairs@, SW_REC = @record@, SW_NBY = @nby@;
    const long long _s_t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (_s_t >= (long long)@slots@) return;
    const int _s_lane = (int)(_s_t & 63);
    const long long _s_row = _s_t >> 6;                 // bundle * SW_SPA + step
    const int _s_step = (int)(_s_row % SW_SPA), _s_beta = (int)(_s_row / SW_SPA);
    const int _s_y = (_s_beta % SW_NBY) * SW_WY + _s_lane % SW_WY;
    const int _s_z = (_s_beta / SW_NBY) * SW_WZ + _s_lane / SW_WY;
    const int _s_x = _s_step - _s_lane % SW_WY - SW_SKZ * (_s_lane / SW_WY);
    const bool _s_active = _s_x >= 0 && _s_x < SW_NX && _s_y < SW_NY && _s_z < SW_NZ;
    @it@ = _s_active ? (lcd_index_t)(_s_x + SW_NX * (_s_y + (long long)SW_NY * _s_z)) : 0;
    double* const _s_rec = _lcd_sw_ops + _s_row * SW_REC;      // the step's record
    (void)_s_rec; (void)_lane;
"""


_SWEEP_TILE = r"""
    // one workgroup of 256 threads per tile of 32 steps x 64 lanes of a bundle:
    // memory is touched in runs along the grid lines on one side and along the
    // lanes of a record on the other, the tile turns in LDS between the two
    constexpr int SW_NX = @nx@, SW_NY = @ny@, SW_NZ = @nz@, SW_WY = @wy@, SW_WZ = @wz@;
    constexpr int SW_SKZ = @skz@, SW_SPA = @spa@, SW_P = @pairs@, SW_REC = @record@, SW_NBY = @nby@;
    constexpr int SW_TS = @tile_steps@;
    const int _s_beta = (int)(blockIdx.x / (SW_SPA / SW_TS));
    const int _s_s0 = (int)(blockIdx.x % (SW_SPA / SW_TS)) * SW_TS;
    const int _s_by = _s_beta % SW_NBY, _s_bz = _s_beta / SW_NBY;
    const long long _s_row0 = (long long)_s_beta * SW_SPA + _s_s0;
    (void)_lane; (void)_s_row0;
    // (lane of the bundle, step of the tile) -> is there a task, and which
    auto _s_task = [&](int lane, int st, bool& active) {
        const int y = _s_by * SW_WY + lane % SW_WY, z = _s_bz * SW_WZ + lane / SW_WY;
        const int x = _s_s0 + st - lane % SW_WY - SW_SKZ * (lane / SW_WY);
        active = x >= 0 && x < SW_NX && y < SW_NY && z < SW_NZ;
        return active ? (lcd_index_t)(x + SW_NX * (y + (long long)SW_NY * z)) : (lcd_index_t)0;
    };
"""


class GridSweepMixin:
    """Methods of ``HIPLowerer`` (lcd_amd/hip_lowering.py)."""

    def _sweep_parts(self, task_lines):
        """The task's text split the way the walkers split it -- what the
        staging kernels evaluate per task (node loads, the element's first
        value) and what the sweeping wavefront runs per step (the tail) --
        with the components of a step's record, or None when the task does
        not fit: an arithmetic tail over +, -, * and the one prepared
        division, so that a lane without a task, which computes on ones,
        never makes a value that is no number."""
        plan, box = self._walker, self._mailbox
        gather, register = box["gather"], box["register"]
        split = plan.get("split", 0) if box.get("pulled") else 0
        head_lines, tail_lines = task_lines[:split], task_lines[split:]
        assign = re.compile(r"^(\w+) = (.*);$")
        stage_lines, staged, zero_start = [], [], False
        for line in self._prefetch_lines:
            match = assign.match(line.strip())
            if match is None:
                return None
            if match.group(1) == register:
                if match.group(2) != "0.0":
                    return None
                zero_start = True
                continue
            stage_lines.append(line.strip())
            staged.append(match.group(1))
        if not head_lines and not zero_start:
            return None
        head = []
        for line in head_lines:
            match = assign.match(line.strip())
            if match is None:
                return None
            head.append(line.strip())
            if match.group(1) != register:
                staged.append(match.group(1))
        tail_text = "\n".join(tail_lines)
        plain = tail_text.replace("_lcd_wdiv(", "(")
        if "/" in plain or "%" in plain or re.search(r"\b(?!if\b|for\b|while\b)[A-Za-z_]\w*\s*\(", plain):
            return None
        slots = [(name, self._kinds.locals.get(name, FLOAT))
                 for name in dict.fromkeys(staged)
                 if re.search(r"\b" + re.escape(name) + r"\b", tail_text)]
        division = plan["division"]
        if division:
            slots.append(("_lcd_wr", FLOAT))
        if head:
            slots.append((register, FLOAT))
        # which of them change with the matrix values only: everything the
        # staging computes from integer arrays and the arrays of the product's
        # operand; the rest (the right-hand side) is staged before every solve
        arrays = self._kinds.arrays
        static_arrays = {name for name, kind in arrays.items() if kind == INT}
        _, operand_node, _ = gather["operands"][0]
        static_arrays |= {node.value.id for node in ast.walk(operand_node)
                          if isinstance(node, ast.Subscript)
                          and isinstance(node.value, ast.Name)}
        dynamic = set()
        for line in stage_lines + head:
            name, text = assign.match(line).groups()
            words = set(re.findall(r"[A-Za-z_]\w*", text))
            if any(word in arrays and word not in static_arrays for word in words) or (
                    words & dynamic):
                dynamic.add(name)
        if division and division in dynamic:
            dynamic.add("_lcd_wr")
        entries = 3
        ordered = ([slot for slot in slots if slot[0] not in dynamic]
                   + [slot for slot in slots if slot[0] in dynamic])
        return {
            "head": head, "tail": tail_lines, "stage": stage_lines,
            "slots": ordered, "dynamic": dynamic, "division": division,
            "entries": entries, "components": entries + len(ordered),
            "start": (entries + [n for n, _ in ordered].index(register)
                      if head else None),
            "static_arrays": tuple(sorted(
                name for name in static_arrays if arrays.get(name) == FLOAT)),
        }

    def _sweep_component(self, c):
        """Component ``c`` of step ``j``'s record in the sweeping wavefront's
        registers."""
        pairs = self._sweep["geometry"]["pairs"]
        if c >= 2 * pairs:
            return f"lcd_whole(_s_h[j][{c - 2 * pairs}])"
        return (f"lcd_lo(_s_o[j][{c // 2}])" if c % 2 == 0
                else f"lcd_hi(_s_o[j][{c // 2}])")

    def _sweep_record_slot(self, c, lane):
        """Where component ``c`` of lane ``lane`` lies in a step's record
        (``_s_rec``): in a plane of pairs, or in a plane of its own."""
        pairs = self._sweep["geometry"]["pairs"]
        if c >= 2 * pairs:
            return f"_s_rec[{pairs * 128 + (c - 2 * pairs) * 64} + {lane}]"
        return f"_s_rec[{(c // 2) * 128 + c % 2} + {lane} * 2]"

    def _grid_sweep_text(self, task_lines):
        """Kernel body of the sweep (everything after the declarations)."""
        parts = self._sweep_parts(task_lines)
        if parts is None:
            return None
        self._sweep = parts
        geometry = sweep_geometry(
            self.grid_sweep[:3], *self.grid_sweep[3:],
            components=parts["components"],
            dynamic=sum(1 for slot in parts["slots"]
                        if slot[0] in parts["dynamic"]))
        if geometry["lds_bytes"] > LDS_BYTES or (
                self.threads_per_block != geometry["threads"]):
            return None
        parts["geometry"] = geometry
        box = self._mailbox
        gather, register = box["gather"], box["register"]
        emitter = self._emitter
        operand = gather["operands"][0][0]
        sign = "-" if gather["negate"] else "+"
        product = emitter.expr(gather["value"])
        pad = " " * 16
        take = [f"{pad}{register} = "
                + (self._sweep_component(parts["start"])
                   if parts["start"] is not None else "0.0") + ";"]
        for k, (name, kind) in enumerate(parts["slots"]):
            if name == register:
                continue
            what = self._sweep_component(parts["entries"] + k)
            take.append(f"{pad}{name} = (lcd_index_t){what};" if kind == INT
                        else f"{pad}{name} = {what};")
        if re.search(r"\b" + re.escape(self.loop_iterator) + r"\b",
                     "\n".join(parts["tail"])):
            # (the tail names the task: its place on the lane's line)
            take.append(
                f"{pad}{self.loop_iterator} = (lcd_index_t)(s0 + j - ly - SW_SKZ * lz"
                " + SW_NX * ((_s_by * SW_WY + ly) + (long long)SW_NY * "
                "(_s_bz * SW_WZ + lz)));")
        if geometry["wy"] == 16:
            vy = [f"{pad}const double _s_vy = lcd_row_shr1_or(fy_now, _s_prev);"]
        else:
            vy = [f"{pad}const double _s_vy = lcd_row_shr1_sel(fy_now, _s_prev, ly == 0);"]
        task = []
        for k, value in enumerate(("_s_vz", "_s_vy", "_s_prev")):
            task += [f"{pad}_g_value = {value}; {operand} = "
                     f"{self._sweep_component(k)};",
                     f"{pad}{register} = {register} {sign} {product};"]
        task += [pad + line for line in parts["tail"]]
        text = _SWEEP_KERNEL
        values = dict(geometry, depth=SWEEP_DEPTH, operand=operand,
                      take="\n".join(take), vy="\n".join(vy),
                      task="\n".join(task))
        for key, value in values.items():
            text = text.replace(f"@{key}@", str(value))
        return text.strip("\n").split("\n")

    def _grid_stage_kernels(self, function_name, signature, declarations):
        """The three kernels around the sweep: what a step's record holds of
        the matrix arrays (``..._sweep_static``), what it holds of the other
        arrays (``..._sweep_dynamic``), and the solution back to its array
        (``..._sweep_unstage``).  One thread per (bundle, step, lane)."""
        parts, box = self._sweep, self._mailbox
        geometry = parts["geometry"]
        gather = box["gather"]
        emitter = self._emitter
        operand, operand_node, _ = gather["operands"][0]
        neutral = "-0.0" if not gather["negate"] else "0.0"
        it = self.loop_iterator
        head = _SWEEP_SLOT
        for key, value in dict(geometry, it=it).items():
            head = head.replace(f"@{key}@", str(value))
        names = tuple(f"{function_name}_hip_sweep_{kind}"
                      for kind in ("static", "dynamic", "unstage"))

        def component(c, lane="_s_lane"):
            return self._sweep_record_slot(c, lane)

        def put(name, kind):
            return f"(double){name}" if kind == INT else name

        assign = re.compile(r"^(\w+) = (.*);$")
        static_lines = [line for line in parts["stage"] + parts["head"]
                        if assign.match(line).group(1) not in parts["dynamic"]]
        all_lines = parts["stage"] + parts["head"]
        division = parts["division"]
        reciprocal = ([f"_lcd_wr = lcd_div_plain_divisor({division}) ? "
                       f"lcd_div_prepare({division}) : lcd_empty();"]
                      if division else [])
        entries = parts["entries"]

        def kernel(name, body):
            return [f'extern "C" __global__ void {name}(',
                    f"        {signature})", "{",
                    "    const int _lane = 0;", f"    lcd_index_t {it} = 0;",
                    *declarations,
                    *(["    double _lcd_wr = 0.0; (void)_lcd_wr;"]
                      if division else []),
                    "    lcd_index_t _g_pos = 0, _g_src = 0; (void)_g_pos; (void)_g_src;",
                    f"    double {operand} = 0.0; (void){operand};",
                    *head.strip("\n").split("\n"), *body, "}", ""]

        static_slots = [(k, slot) for k, slot in enumerate(parts["slots"])
                        if slot[0] not in parts["dynamic"]]
        dynamic_slots = [(k, slot) for k, slot in enumerate(parts["slots"])
                         if slot[0] in parts["dynamic"]]
        static_body = [
            f"    double _s_c[{entries}];",
            f"    for (int k = 0; k < {entries}; ++k) _s_c[k] = {neutral};",
            "    if (_s_active) {",
            "        // the incoming entries by direction: one step down along z, y, x",
            f"        for (int e = _lcd_in_ptr[{it}]; e < _lcd_in_ptr[{it} + 1]; ++e) {{",
            "            _g_src = (lcd_index_t)_lcd_in_src[e]; _g_pos = (lcd_index_t)_lcd_in_pos[e];",
            f"            const long long d = (long long){it} - _g_src;",
            "            const int k = d == (long long)SW_NX * SW_NY ? 0 : d == SW_NX ? 1 : d == 1 ? 2 : -1;",
            f"            if (k < 0) _lcd_status[0] = 3; else _s_c[k] = {emitter.expr(operand_node)};",
            "        }",
            *["        " + line for line in static_lines],
            *(["        " + line for line in reciprocal]
              if division and "_lcd_wr" not in parts["dynamic"] else []),
            "    }",
            *[f"    {component(k)} = _s_c[{k}];" for k in range(entries)],
            # (a lane without a task computes on ones)
            *[f"    {component(entries + k)} = _s_active ? {put(name, kind)} : 1.0;"
              for k, (name, kind) in static_slots],
            # (the unused half of an odd last plane of pairs does not exist:
            # an odd component has a plane of 8-byte slots)
        ]
        tile_head = _SWEEP_TILE
        for key, value in dict(geometry, tile_steps=SWEEP_TILE_STEPS).items():
            tile_head = tile_head.replace(f"@{key}@", str(value))

        def tile_kernel(name, body):
            return [f'extern "C" __global__ void __launch_bounds__(256) {name}(',
                    f"        {signature})", "{",
                    "    const int _lane = 0;", f"    lcd_index_t {it} = 0;",
                    *declarations,
                    *(["    double _lcd_wr = 0.0; (void)_lcd_wr;"]
                      if division else []),
                    *tile_head.strip("\n").split("\n"), *body, "}", ""]

        count = max(len(dynamic_slots), 1)
        dynamic_body = [
            f"    __shared__ double _s_tile[{count}][SW_TS][65];",
            f"    double _s_v[{count}][8];",
            # (a slot without a task reads task 0's operands, so that the
            # eight passes' loads are all under way together, and computes
            # on ones)
            "    _Pragma(\"unroll\") for (int p = 0; p < 8; ++p) {",
            "        const int lane = p * 8 + (int)(threadIdx.x >> 5), st = (int)(threadIdx.x & 31);",
            "        bool active;",
            f"        {it} = _s_task(lane, st, active);",
            *["        " + line for line in all_lines],
            *(["        " + line for line in reciprocal]
              if division and "_lcd_wr" in parts["dynamic"] else []),
            *[f"        _s_v[{q}][p] = active ? {put(name, kind)} : 1.0;"
              for q, (k, (name, kind)) in enumerate(dynamic_slots)],
            "    }",
            "    _Pragma(\"unroll\") for (int p = 0; p < 8; ++p) {",
            "        const int lane = p * 8 + (int)(threadIdx.x >> 5), st = (int)(threadIdx.x & 31);",
            *[f"        _s_tile[{q}][st][lane] = _s_v[{q}][p];"
              for q in range(len(dynamic_slots))],
            "    }",
            "    __syncthreads();",
            "    for (int u = 0; u < 8; ++u) {",
            "        const int at = u * 256 + (int)threadIdx.x, st = at >> 6, lane = at & 63;",
            "        double* const _s_rec = _lcd_sw_ops + (_s_row0 + st) * SW_REC;",
            *[f"        {component(entries + k, 'lane')} = _s_tile[{q}][st][lane];"
              for q, (k, _) in enumerate(dynamic_slots)],
            "    }",
        ]
        unstage_body = [
            "    __shared__ double _s_tile[SW_TS][65];",
            "    for (int u = 0; u < 8; ++u) {",
            "        const int at = u * 256 + (int)threadIdx.x, st = at >> 6, lane = at & 63;",
            "        _s_tile[st][lane] = _lcd_sw_out[(_s_row0 + st) * 64 + lane];",
            "    }",
            "    __syncthreads();",
            "    for (int p = 0; p < 8; ++p) {",
            "        const int lane = p * 8 + (int)(threadIdx.x >> 5), st = (int)(threadIdx.x & 31);",
            "        bool active;",
            f"        {it} = _s_task(lane, st, active);",
            f"        if (active) {box['array']}[{it}] = _s_tile[st][lane];",
            "    }",
        ]
        lines = (kernel(names[0], static_body)
                 + tile_kernel(names[1], dynamic_body)
                 + tile_kernel(names[2], unstage_body))
        self._sweep["kernels"] = names
        self._sweep["dynamic_kernel"] = bool(dynamic_slots)
        return "\n".join(lines) + "\n"
