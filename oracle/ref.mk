# placeholder until the reference build recipe lands
ref:
