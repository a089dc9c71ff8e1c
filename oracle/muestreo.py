"""CPU restatement of the generation loop's per-token choice -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

What the reference's escribir does to the logits before its multinomial draw, in float64 on the CPU:
  ngramas_siguientes   the tokens that close an n-gram already in a text: _Ngramas (asrn/nucleo.py:1857-1889), as
                       sets of token tuples, and the direct search over the text (_continuaciones_de_cita,
                       nucleo:1921-1930; _frenos' ban branch, nucleo:1892-1906) beside it
  frenar               the repetition penalty and the bans (_frenar, nucleo:1909-1918) with the fallback when every
                       token is banned (nucleo:2020-2021)
  probabilidades       temperature, top-k, top-p by sorting (_muestrear, nucleo:1946-1961) and _conservar_cita
                       (nucleo:1933-1943): the distribution the draw samples from
Pinned in tests/test_oracle_sampling.py by the reference's own tests of these functions (tests/test_nucleo.py:
590-635 and 1237-1248: top_p = 0 keeps the most probable, the quote mass stays the temperature-1 mass, the shape
inside each part is q's) and by the direct definitions (sets against the text search, top-k against a sort).
"""
import torch


def ngramas_siguientes(texto, n):
    """Set of tokens v such that texto[-(n-1):] + [v] is an n-gram of texto (the sets of _Ngramas.siguientes); empty
    while len(texto) < n."""
    if len(texto) < n:
        return set()
    mapa = {}
    for i in range(n - 1, len(texto)):
        mapa.setdefault(tuple(texto[i - n + 1:i]), set()).add(texto[i])
    return set(mapa.get(tuple(texto[len(texto) - n + 1:]), ()))


def ngramas_siguientes_directo(texto, n):
    """The same set by scanning every window of the text (the definition _continuaciones_de_cita and _frenos use)."""
    if len(texto) < n:
        return set()
    cola = texto[len(texto) - (n - 1):] if n > 1 else []
    return {texto[s + n - 1] for s in range(len(texto) - n + 1) if texto[s:s + n - 1] == cola}


def frenar(lg, texto, L0, pena, ventana, no_repetir):
    """lg (V,) float64 and one text (a list, prompt then generated) -> the logits after the penalty over the last
    `ventana` tokens and the ban of tokens closing an n-gram of the generated part; all banned -> lg unchanged."""
    lg = lg.clone()
    out = lg.clone()
    if pena != 1.0:
        for v in set(texto[max(0, len(texto) - ventana):]):
            out[v] = out[v] / pena if lg[v] > 0 else lg[v] * pena
    if no_repetir:
        for v in ngramas_siguientes(texto[L0:], no_repetir):
            out[v] = -float('inf')
    if torch.isneginf(out).all():
        return lg
    return out


def probabilidades(lg, temperatura, top_k, top_p, cita=None):
    """lg (V,) float64 after frenar, cita a set of token ids or None -> the probabilities the draw uses."""
    V = lg.shape[0]
    p1 = torch.softmax(lg, -1)
    x = lg / max(temperatura, 1e-6)
    if top_k and top_k < V:
        corte = torch.sort(x, descending=True).values[top_k - 1]
        x = torch.where(x < corte, torch.full_like(x, -float('inf')), x)
    if top_p < 1.0:
        orden, idx = torch.sort(x, descending=True, stable=True)
        p = torch.softmax(orden, -1)
        antes = torch.cumsum(p, -1) - p
        fuera = antes >= top_p
        fuera[0] = False
        x = x.clone()
        x[idx[fuera]] = -float('inf')
    q = torch.softmax(x, -1)
    if cita:
        m = torch.zeros(V, dtype=torch.bool)
        m[list(cita)] = True
        masa_p, masa_q = p1[m].sum(), q[m].sum()
        if 0 < masa_q < 1:
            q = torch.where(m, q * masa_p / masa_q, q * (1 - masa_p) / (1 - masa_q))
    return q
