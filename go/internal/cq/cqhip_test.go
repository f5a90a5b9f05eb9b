//go:build cqhip

// Tests of the cqhip build of package cq through its public API only (the
// CPU build's tests reach into its kernels and stay behind !cqhip). Not
// compiled in the repository that ships it; the same properties are
// checked there through the C ABI (tests/test_gpu_cq.py, tests/test_abi.py).
package cq

import (
	"encoding/binary"
	"math"
	"math/rand/v2"
	"slices"
	"strings"
	"testing"

	"github.com/cwbudde/go-whistle/internal/cact"
)

// synthPacked returns an out x in CQ tensor of `bits` for these tests:
// every index value drawn on its own, uniform over the 2^bits codes, and
// packed LSB first into its row's bytes (the layout cact.Packed documents,
// internal/cact/packed.go:18-40); 2^bits levels mirrored about zero with
// magnitudes |N(0, 1/group)|, sorted; FP16 norms of 2^-4 .. 2^4.
func synthPacked(rng *rand.Rand, out, in, group, bits int) cact.Packed {
	p := cact.Packed{Out: out, In: in, Group: group, Bits: bits, Width: bits}
	sigma := 1 / math.Sqrt(float64(group))
	levels := make([]float32, 0, 1<<bits)
	for range 1 << (bits - 1) {
		m := float32(math.Abs(rng.NormFloat64()) * sigma)
		levels = append(levels, m, -m)
	}
	slices.Sort(levels)
	p.Codebook = levels

	rowBytes, perByte := p.RowBytes(), 8/bits
	p.Index = make([]byte, out*rowBytes)
	for r := range out {
		row := p.Index[r*rowBytes : (r+1)*rowBytes]
		for k := range rowBytes * perByte {
			code := byte(rng.IntN(1 << bits))
			row[k/perByte] |= code << (uint(k%perByte) * uint(bits))
		}
	}

	p.Norms = make([]byte, 2*out*p.Groups())
	for i := 0; i < len(p.Norms); i += 2 {
		exp := uint16(11 + rng.IntN(9)) // biased exponent: 2^-4 .. 2^4
		binary.LittleEndian.PutUint16(p.Norms[i:], exp<<10|uint16(rng.IntN(1<<10)))
	}

	return p
}

func normals(rng *rand.Rand, n int) []float32 {
	x := make([]float32, n)
	for i := range x {
		x[i] = float32(rng.NormFloat64())
	}

	return x
}

// dense returns row r of W·x in float64 from Row's dequantised weights, and
// the scale Σ|w·x| its rounding errors are measured against.
func dense(m *Matrix, x []float32, r int) (y, scale float64) {
	w := make([]float32, m.In())
	m.Row(w, r)

	for i, v := range w {
		y += float64(v) * float64(x[i])
		scale += math.Abs(float64(v) * float64(x[i]))
	}

	return y, scale
}

func TestCQHIPProducts(t *testing.T) {
	for _, s := range []struct{ out, in, bits int }{{96, 512, 2}, {384, 512, 2}, {128, 2048, 4}, {8199, 512, 4}} {
		rng := rand.New(rand.NewPCG(uint64(s.out), uint64(s.in)))

		m, err := New(synthPacked(rng, s.out, s.in, 128, s.bits))
		if err != nil {
			t.Fatal(err)
		}

		x := normals(rng, s.in)
		lut := make([]float32, s.out)
		exact := make([]float32, s.out)
		m.GEMV(lut, x)
		m.Exact().GEMV(exact, x)

		for r := range s.out {
			want, scale := dense(m, x, r)
			// nibble4 sums the levels in float32; the lut kernel rounds its
			// tables to 14-bit integers (lut.go:16-27)
			if d := math.Abs(float64(exact[r]) - want); d > 1e-5*scale {
				t.Fatalf("%dx%d CQ%d row %d: exact %v, dense %v (scale %v)", s.out, s.in, s.bits, r, exact[r], want, scale)
			}

			if d := math.Abs(float64(lut[r]) - want); d > 2e-3*scale {
				t.Fatalf("%dx%d CQ%d row %d: lut %v, dense %v (scale %v)", s.out, s.in, s.bits, r, lut[r], want, scale)
			}
		}
	}
}

func TestCQHIPBatchesAndViews(t *testing.T) {
	rng := rand.New(rand.NewPCG(3, 4))
	p := synthPacked(rng, 4*512, 512, 128, 4)

	m, err := New(p)
	if err != nil {
		t.Fatal(err)
	}

	const rows = 5
	x := normals(rng, rows*512)
	y := make([]float32, rows*m.Out())
	m.GEMM(y, x, rows)

	// each row of a GEMM is that activation's GEMV, bit for bit
	for r := range rows {
		g := make([]float32, m.Out())
		m.GEMV(g, x[r*512:(r+1)*512])

		if !slices.Equal(g, y[r*m.Out():(r+1)*m.Out()]) {
			t.Fatalf("GEMM row %d differs from its GEMV", r)
		}
	}

	// row views and GEMMs over them give the root's rows, bit for bit
	spans := [][2]int{{0, 512}, {512, 1024}, {1024, 1500}, {1500, 2048}}
	views := make([]*Matrix, len(spans))
	dsts := make([][]float32, len(spans))

	for k, sp := range spans {
		views[k] = m.Rows(sp[0], sp[1])
		dsts[k] = make([]float32, rows*(sp[1]-sp[0]))
	}

	GEMMs(views, dsts, x, rows)

	for k, sp := range spans {
		n := sp[1] - sp[0]
		for r := range rows {
			if !slices.Equal(dsts[k][r*n:(r+1)*n], y[r*m.Out()+sp[0]:r*m.Out()+sp[1]]) {
				t.Fatalf("view %v row %d differs from the root's rows", sp, r)
			}
		}
	}

	if m.Bytes() <= 0 || views[0].Out() != 512 || views[0].In() != 512 || views[0].Bits() != 4 {
		t.Fatalf("shape or bytes: %d %d %d %d", m.Bytes(), views[0].Out(), views[0].In(), views[0].Bits())
	}
}

func TestCQHIPNewErrors(t *testing.T) {
	good := synthPacked(rand.New(rand.NewPCG(7, 8)), 2, 128, 128, 2)

	for _, tc := range []struct {
		name string
		edit func(p *cact.Packed)
		want string
	}{
		{"3 bits", func(p *cact.Packed) { p.Bits, p.Width = 3, 3 }, "not supported"},
		{"ternary", func(p *cact.Packed) { p.Bits = 5 }, "not supported"},
		{"group 24", func(p *cact.Packed) { p.Group = 24 }, "power of two"},
		{"codebook", func(p *cact.Packed) { p.Codebook = p.Codebook[:3] }, "codebook"},
		{"index", func(p *cact.Packed) { p.Index = p.Index[1:] }, "index"},
		{"norms", func(p *cact.Packed) { p.Norms = p.Norms[2:] }, "norm"},
	} {
		p := good
		tc.edit(&p)

		if _, err := New(p); err == nil || !strings.Contains(err.Error(), tc.want) {
			t.Errorf("%s: err = %v, want one mentioning %q", tc.name, err, tc.want)
		}
	}
}

func TestCQHIPPanics(t *testing.T) {
	m, err := New(synthPacked(rand.New(rand.NewPCG(9, 10)), 4, 128, 128, 4))
	if err != nil {
		t.Fatal(err)
	}

	for name, f := range map[string]func(){
		"short x":   func() { m.GEMV(make([]float32, 4), make([]float32, 127)) },
		"short dst": func() { m.GEMV(make([]float32, 3), make([]float32, 128)) },
		"rows":      func() { m.GEMM(make([]float32, 8), make([]float32, 128), 2) },
		"row":       func() { m.Row(make([]float32, 128), 4) },
		"view":      func() { m.Rows(3, 5) },
	} {
		func() {
			defer func() {
				if recover() == nil {
					t.Errorf("%s: no panic", name)
				}
			}()

			f()
		}()
	}
}
